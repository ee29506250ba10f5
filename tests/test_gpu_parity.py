"""GPU parity: libdmc_hip (through its C ABI) against the CPU oracle.

Every case runs the same seeded inputs through the device and through the
oracle (the reference's dmc_matmul_bf16 chain, compiler/src/jit.rs:29481-29681)
and applies tests/parity.py's rule.  Layouts: "rd" goes through
dmc_matmul_bf16_gpu_t (row-dot kernels on W [N,K]); "cs" through the drop-in
dmc_matmul_bf16_gpu (x @ W with W [K,N], which a single slice serves with the
row-dot kernels on a transposed resident copy); "cs_dev" through
dmc_hip_gemv_cs on device pointers (the column-stream kernels).  Batched and
deferred calls run the column-stream kernels too.
"""
import numpy as np
import pytest

import oracle
from demonic_amd import workloads as W
from parity import check, check_bound, check_or_bound

pytestmark = pytest.mark.gpu


def case(m, k, n, seed, edge=False, scale=1.0):
    """x [m,k] f32 and logical w [n,k] bf16; `edge` adds subnormals, +-0,
    +-1e-38 in x and a few inf/NaN weights."""
    rng = np.random.Generator(np.random.PCG64(seed))
    w = W.bf16_rne(np.float32(scale) * rng.standard_normal((n, k), dtype=np.float32))
    x = rng.standard_normal((m, k), dtype=np.float32)
    if edge and k > 0 and n > 0:
        cnt = max(1, n * k // 200)
        flat = w.reshape(-1)
        pos = rng.integers(0, n * k, size=cnt)
        flat[pos] = (rng.integers(0, 2, size=cnt, dtype=np.uint16) << 15) | \
            rng.integers(1, 128, size=cnt, dtype=np.uint16)
        xs = x.reshape(-1)
        pos = rng.integers(0, xs.size, size=max(1, xs.size // 20))
        xs[pos] = rng.choice(np.array([0.0, -0.0, 1e-38, -1e-38], np.float32), size=pos.size)
        if n * k >= 64:
            pos = rng.integers(0, n * k, size=3)
            flat[pos] = np.array([0x7F80, 0xFF80, 0x7FC0], np.uint16)
    return x, w


def run_rd(hip, x, w):
    return hip.matmul_bf16_gpu_t(x, w)


def run_cs(hip, x, w):
    return hip.matmul_bf16_gpu(x, np.ascontiguousarray(w.T))


def run_cs_dev(hip, x, w):
    """x @ W' through the column-stream kernels on device pointers (W^T [K,N] in HBM)."""
    x = np.ascontiguousarray(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    m, k = x.shape
    n = w.shape[0]
    wt = np.ascontiguousarray(w.T)
    with hip.DeviceBuffer.from_numpy(wt if wt.size else np.zeros(1, np.uint16)) as dw, \
            hip.DeviceBuffer.from_numpy(x if x.size else np.zeros(1, np.float32)) as dx, \
            hip.DeviceBuffer(max(4, 4 * m * n)) as dy:
        hip.gemv_cs(dx, dw, dy, m, k, n)
        hip.synchronize()
        return dy.download(np.float32, (m, n))


RUN = {"rd": run_rd, "cs": run_cs, "cs_dev": run_cs_dev}
LAYOUTS = list(RUN)


def ref(x, w):
    return oracle.matmul_bf16_t(x, w)


# ---- basic facts ----------------------------------------------------------------------

def test_device_is_gfx950(hip):
    info = hip.device_info()
    assert info["arch"] == "gfx950", info
    assert info["cus"] > 0


def test_denormals_survive_and_inf_times_tiny_is_inf(hip):
    # 1e-38 is an f32 subnormal; flushing it would turn 1e-38 * inf into NaN.
    k = 1000
    x = np.zeros((1, k), np.float32)
    x[0, 5] = np.float32(1e-38)
    w = np.zeros((3, k), np.uint16)
    w[0, 5] = 0x7F80          # +inf
    w[1, 5] = 0x3F80          # 1.0  -> y = 1e-38 exactly
    w[2, :] = 0x0001          # smallest bf16 subnormal everywhere
    x2 = x.copy()
    x2[0, :] = 1.0
    for run in RUN.values():
        y = run(hip, x, w)[0]
        assert np.isposinf(y[0]), y
        assert y[1] == np.float32(1e-38), y
        y2 = run(hip, x2, w)[0]
        assert y2[2] == np.float32(k) * W.bf16_to_f32(np.array([1], np.uint16))[0], y2


@pytest.mark.parametrize("kind", [6, 7, 8])
@pytest.mark.parametrize("m,k", [(2, 64), (3, 320), (4, 4096), (8, 1024), (16, 64)])
def test_skinny_mfma_underflowing_products_keep_their_zero_sign(hip, m, k, kind, monkeypatch):
    """As the M = 1 case above, through each MFMA layout: weight row 0's
    products all underflow negative (reference -0.0), row 1's positive (+0.0),
    row 2 is exact zeros against negative x (products -0.0, reference +0.0).
    K = 64 leaves seven of rows16's eight waves without a line: they add -0.0."""
    x = np.full((m, k), np.float32(-1e-38), np.float32)
    w = np.zeros((3, k), np.uint16)
    w[0, :] = 0x0001
    w[1, :] = 0x8001
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", str(kind))
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "2")  # M = 2 included
    assert hip.plan("rd", m, k, 3, x_addr=x.ctypes.data, w_addr=w.ctypes.data).slices == -kind
    y_ref = ref(x, w)
    assert np.all(np.signbit(y_ref[:, 0])) and not np.any(np.signbit(y_ref[:, 1:]))
    y = run_rd(hip, x, w)
    check(y, y_ref, what=f"mfma underflow signs m={m} k={k} kind={kind}")


@pytest.mark.parametrize("kind", [6, 7, 8])
def test_skinny_mfma_zero_outputs_follow_the_reference_chain(hip, kind, monkeypatch):
    """An MFMA output that comes out exactly zero is settled by the reference's
    own chain, so even the order-dependent zeros match bit for bit: rows whose
    underflowing products change sign along k (the chain keeps the sign of the
    last one, then +-0 products may flip -0 to +0), exact cancellation, and
    all-zero weight and activation rows."""
    m, k = 4, 256
    x = np.full((m, k), np.float32(1e-38), np.float32)
    x[1] = -x[1]
    x[3] = 0                                   # an all-zero activation row
    x[2, ::3] = -x[2, ::3]
    w = np.full((8, k), 0x0001, np.uint16)     # every product underflows
    w[1, k - 1] = 0x8001                       # last product flips sign
    w[2, k - 1] = 0x0000                       # then a +-0 product after the last nonzero one
    w[3, 1::2] = 0x8001                        # alternating signs
    w[4] = 0                                   # an all-zero weight row
    w[5, :] = 0x3F80                           # 1.0 ...
    w[5, k // 2:] = 0xBF80                     # ... and -1.0: exact cancellation against x = 1e-38
    w[6, :7] = 0x8001
    w[7, ::5] = 0x8000                         # -0 weights among positive tiny products
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", str(kind))
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "2")  # M = 2 included
    assert hip.plan("rd", m, k, 8, x_addr=x.ctypes.data, w_addr=w.ctypes.data).slices == -kind
    y_ref = ref(x, w)
    assert np.any(np.signbit(y_ref[y_ref == 0])) and np.any(~np.signbit(y_ref[y_ref == 0]))
    y = run_rd(hip, x, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), (y, y_ref)


@pytest.mark.parametrize("tiles", [2, 4])
@pytest.mark.parametrize("m", [2, 5, 8, 16])
def test_rows16_blocks_per_workgroup(hip, m, tiles, monkeypatch):
    """rows16 with 2 or 4 16-row blocks per workgroup, gridDim.x blocks apart:
    N = 40003 leaves a 3-row block and, at 4 blocks, three empty ones.  Edge
    data (subnormals, +-0, +-1e-38, inf/NaN weights), an all-zero weight row,
    rows sampled from every block position and the last rows."""
    k, n = 1024, 40003
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "7")
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "2")  # M = 2 included
    monkeypatch.setenv("DMC_HIP_RD_R16_TILES", str(tiles))
    x, w = case(m, k, n, seed=77 + m * 5 + tiles, edge=True)
    w[n - 2, :] = 0
    p = hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert (p.slices, p.rows_per_group) == (-7, 16 * tiles), p
    y = run_rd(hip, x, w)
    rng = np.random.default_rng(m)
    rows = np.unique(np.r_[np.arange(n - 40, n), np.arange(0, 48), rng.integers(0, n, 400),
                           np.array([16 * p.grid_x, 16 * p.grid_x + 15, 32 * p.grid_x - 1]) % n])
    y_ref = oracle.matmul_bf16_t(x, w[rows])
    check(y[:, rows], y_ref, what=f"rows16 m={m} tiles={tiles}")
    assert np.all(y[:, n - 2][np.isfinite(y_ref[:, list(rows).index(n - 2)])] == 0)


# ---- shape and tail coverage ----------------------------------------------------------

SHAPES = [
    (1, 1, 1), (1, 7, 3), (1, 8, 5), (1, 63, 64), (1, 64, 65), (1, 65, 129),
    (1, 511, 7), (1, 512, 8), (1, 513, 9), (1, 1000, 33), (1, 2048, 1), (1, 4097, 37),
    (2, 64, 17), (3, 129, 31), (5, 1024, 100), (8, 520, 24), (16, 4096, 40),
    (17, 300, 11), (33, 96, 65), (1, 12288, 6),
    # misaligned rows with a short tail past whole blocks of windows: one
    # element (4097), two (4098), seven (4103, 8199, 12295: one, two and
    # three blocks); aligned rows with eight (4104)
    (1, 4097, 600), (1, 4098, 70), (1, 8199, 300), (1, 12295, 64), (1, 4103, 300), (1, 4104, 301),
]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("layout", LAYOUTS)
def test_shapes(hip, m, k, n, layout):
    x, w = case(m, k, n, seed=1000 + m * 7 + k * 13 + n, edge=True)
    y = RUN[layout](hip, x, w)
    check(y, ref(x, w), what=f"{layout} m={m} k={k} n={n}")


@pytest.mark.parametrize("k,n", [(28672, 600), (28672, 4099), (20480, 1000)])
def test_two_activation_rows_long_rows_on_rows16(hip, k, n):
    """M = 2 on rows too long for the streaming kernel to take both activation
    rows in one pass (k > 16384): rows16 by default (4099 rows: two blocks per
    workgroup and k in two slices).  Edge data; sampled rows within the
    rigorous bound, special classes and zero signs as the reference."""
    x, w = case(2, k, n, seed=8200 + k + n, edge=True)
    p = hip.plan("rd", 2, k, n, x_addr=256, w_addr=256)
    assert p.slices == -7 and p.mt == 4, p
    y = run_rd(hip, x, w)
    rows = np.unique(np.r_[np.arange(0, min(40, n)), np.arange(max(0, n - 40), n),
                           np.random.default_rng(k + n).integers(0, n, 200)])
    y_ref = oracle.matmul_bf16_t(x, w[rows])
    check(y[:, rows], y_ref, what=f"m=2 rows16 k={k} n={n}")
    wf = W.bf16_to_f32(w[rows])
    fin = np.all(np.isfinite(wf), axis=1)
    for r in range(2):
        check_bound(y[r, rows[fin]], y_ref[r, fin], x[r], wf[fin], what=f"m=2 rows16 k={k} n={n} row {r}")


@pytest.mark.parametrize("k,n", [(4096, 14336), (4096, 16387), (14336, 4096), (4096, 40003), (1024, 33), (64, 70)])
def test_two_activation_rows_stream(hip, k, n, monkeypatch):
    """M = 2 on the streaming kernel (its default from 32768 rows; forced here
    with the matrix cores from m = 3) with 16 (or, where the grid would fall
    under 4 workgroups per CU, 8 or 4) weight rows per workgroup: C2's shapes,
    a partial last workgroup (n = 16387, 40003), short rows.  Edge data; every
    element within the rigorous bound, special classes and zero signs as the
    reference."""
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "3")
    x, w = case(2, k, n, seed=8100 + k + n, edge=True)
    p = hip.plan("rd", 2, k, n, x_addr=256, w_addr=256)  # device regions are 256-byte aligned
    assert p.slices > 0 and p.mt == 2, p
    y = run_rd(hip, x, w)
    rows = np.unique(np.r_[np.arange(0, min(40, n)), np.arange(max(0, n - 40), n),
                           np.random.default_rng(k + n).integers(0, n, 300)])
    y_ref = oracle.matmul_bf16_t(x, w[rows])
    check(y[:, rows], y_ref, what=f"m=2 stream k={k} n={n}")
    wf = W.bf16_to_f32(w[rows])
    fin = np.all(np.isfinite(wf), axis=1)
    for r in range(2):
        check_bound(y[r, rows[fin]], y_ref[r, fin], x[r], wf[fin], what=f"m=2 stream k={k} n={n} row {r}")


@pytest.mark.parametrize("offset,k,n", [(2, 4096, 300), (6, 4104, 257), (14, 2048, 33), (10, 777, 1000),
                                        (4, 16384, 70), (2, 11007, 129), (2, 4097, 513), (6, 8192, 129)])
def test_misaligned_weight_view(hip, offset, k, n):
    """W [n,k] starting `offset` bytes into its device region, which ends
    right after the last row: rows on 2-byte boundaries, windows re-aligned
    in registers, the last window's second chunk past the region's end."""
    x, w = case(1, k, n, seed=offset * 31 + k + n, edge=True)
    with hip.DeviceBuffer(offset + w.nbytes) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * n) as dy:
        dw.upload(w, offset=offset)
        hip.gemv_rd(dx.addr, dw.addr + offset, dy, 1, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (1, n))
    check(y, ref(x, w), what=f"view +{offset} k={k} n={n}")


@pytest.mark.parametrize("k", [2450, 2306, 3074])
def test_any_alignment_rowdot_with_waves_past_k_on_device_pointers(hip, k):
    """Rows at 4-byte (not 16-byte) alignment on the any-alignment kernel with
    8 waves, where the last waves' windows all lie past K: x sits in a device
    region of exactly K floats, and its last element is +inf, so a masked
    window that picked up a real x value would turn -0 weights into NaN."""
    n = 567
    rng = np.random.default_rng(k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    x[0, -1] = np.inf
    w = W.bf16_rne(rng.standard_normal((n, k)).astype(np.float32))
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer.from_numpy(w) as dw, \
            hip.DeviceBuffer(4 * n) as dy:
        p = hip.plan("rd", 1, k, n, x_addr=dx.addr, w_addr=dw.addr)
        assert p.vec == 2 and p.slices == 1 and p.waves == 8, p
        hip.gemv_rd(dx, dw, dy, 1, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (1, n))
    check(y, ref(x, w), what=f"any-alignment device k={k}")


@pytest.mark.parametrize("offset,k,n", [(2, 4096, 300), (6, 777, 1000), (2, 11008, 4097), (0, 4097, 4097),
                                        (10, 3, 9), (2, 2, 513)])
def test_column_stream_weight_views_at_any_2_byte_offset(hip, offset, k, n):
    """dmc_hip_gemv_cs on W [k,n] starting `offset` bytes into a region that
    ends right after its last row: the streaming kernel over misaligned rows
    (each row's last chunk runs into the next row; the matrix's last row is
    applied by the slice pass with 2-byte loads, so nothing past the region is
    read)."""
    x, w = case(1, k, n, seed=offset * 7 + k + n, edge=True)
    wkn = np.ascontiguousarray(w.T)
    p = hip.plan("cs", 1, k, n, x_addr=x.ctypes.data, w_addr=256 + offset)
    assert p.rows_or_rw == 0, p
    with hip.DeviceBuffer(offset + wkn.nbytes) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * n) as dy:
        dw.upload(wkn, offset=offset)
        hip.gemv_cs(dx, dw.addr + offset, dy, 1, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (1, n))
    check(y, ref(x, w), what=f"cs view +{offset} k={k} n={n}")


@pytest.mark.parametrize("k", [2, 7, 1000, 4097])
def test_column_stream_misaligned_rows_keep_zero_signs(hip, k):
    """The zero-sign rule of the test below through the streaming kernel over
    odd-N rows: columns whose products all underflow negative end at -0.0,
    positive ones at +0.0, also with the last k row in the slice pass."""
    n = 9
    x = np.full((1, k), np.float32(-1e-38), np.float32)
    w = np.full((n, k), 0x0001, np.uint16)
    w[1::2, :] = 0x8001
    y_ref = ref(x, w)
    assert np.all(np.signbit(y_ref[0, ::2])) and not np.any(np.signbit(y_ref[0, 1::2]))
    y = run_cs_dev(hip, x, w)
    check(y, y_ref, what=f"cs odd-n underflow signs k={k}")


def test_column_stream_batched_slices_at_odd_strides(hip):
    """Batched device calls whose slices start at alternating 2-byte
    alignments (rs and ls odd), N odd."""
    k, n, batch = 300, 1001, 3
    ls, rs = k + 1, k * n + 3
    rng = np.random.default_rng(11)
    x = rng.standard_normal((batch - 1) * ls + k).astype(np.float32)
    w = W.bf16_rne(rng.standard_normal((batch - 1) * rs + k * n).astype(np.float32))
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * batch * n) as dy:
        hip.gemv_cs(dx, dw, dy, 1, k, n, batch, ls, rs)
        hip.synchronize()
        y = dy.download(np.float32, (batch * n,))
    check(y, oracle.matmul_bf16_batched(x, w, k, n, batch, ls, rs), what="cs batched odd strides")


@pytest.mark.parametrize("k,n,batch,per_head,m,groups", [
    (4096, 128, 32, False, 1, 0), (4096, 64, 8, True, 1, 0), (300, 256, 3, True, 3, 0),
    (1001, 136, 4, False, 2, 0), (2048, 1024, 2, True, 1, 8), (7, 128, 5, True, 1, 0), (4096, 8, 16, False, 1, 0),
    (1024, 128, 256, False, 1, 0), (128, 4096, 32, True, 1, 0)])  # k unsplit: a workgroup per CU without it
def test_column_stream_row_groups(hip, k, n, batch, per_head, m, groups, monkeypatch):
    """Batched column-stream calls on narrow N (per-head projections): the
    streaming kernel's wave splits into G row groups of 64/G lanes over
    512/G columns (N = 8, 64 -> G = 8, 128 -> 4, 136 and 256 -> 2), with one
    broadcast x (ls = 0) or one per head, 1..3 activation rows, k shorter
    than one group step, and G = 8 forced on N = 1024 (16 column blocks).
    Edge data, and planted columns whose products all underflow (signs from
    the chain) or are exact zeros; sampled against the oracle within the
    norm and the elementwise bound, zeros bitwise."""
    if groups:
        monkeypatch.setenv("DMC_HIP_CS_ROW_GROUPS", str(groups))
    rng = np.random.default_rng(k * 7 + n + batch)
    x = rng.standard_normal((batch if per_head else 1, m, k)).astype(np.float32)
    w = W.bf16_rne(rng.standard_normal((batch, k, n), dtype=np.float32))
    flat = w.reshape(-1)
    pos = rng.integers(0, flat.size, size=max(1, flat.size // 500))
    flat[pos] = (rng.integers(0, 2, size=pos.size, dtype=np.uint16) << 15) | rng.integers(1, 128, size=pos.size, dtype=np.uint16)
    x[0, 0, :] = np.float32(-1e-38)          # head 0, row 0: tiny x ...
    w[0, :, 0] = 0x0001                      # ... against tiny weights: -0.0
    w[0, :, 1] = 0x8001                      # +0.0
    w[0, :, 2] = 0                           # exact zeros: +0.0
    ls = m * k if per_head else 0
    want_g = groups or next((g for g in (8, 4, 2) if 512 // g >= n), 1)
    p = hip.plan("cs", m, k, n, batch=batch, rs=k * n, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.grid_x) == (-want_g if want_g > 1 else 0, -(-n // (512 // want_g))), p
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * batch * m * n) as dy:
        hip.gemv_cs(dx, dw, dy, m, k, n, batch, ls, k * n)
        hip.synchronize()
        y = dy.download(np.float32, (batch, m, n))
    heads = np.unique(np.r_[0, batch - 1, rng.integers(0, batch, 3)])
    for z in heads:
        xz = x[z if per_head else 0]
        y_ref = oracle.matmul_bf16_t(xz, np.ascontiguousarray(w[z].T))
        check(y[z], y_ref, what=f"cs row groups head {z} k={k} n={n} m={m}")
        wf = W.bf16_to_f32(np.ascontiguousarray(w[z].T))
        fin = np.all(np.isfinite(wf), axis=1)
        for r in range(m):
            check_bound(y[z, r, fin], y_ref[r, fin], xz[r], wf[fin], what=f"cs row groups head {z} row {r}")
        if z == 0:
            assert np.array_equal(y[0, 0, :3].view(np.uint32), y_ref[0, :3].view(np.uint32)), (y[0, 0, :3], y_ref[0, :3])


def zero_rows(k, n=8):
    """Activation rows x [4, k] and weight rows w [n, k] (bf16 bits) whose
    products are all exact zeros or underflow -- so every device sum is
    exactly +-0 and the reference chain decides the sign -- plus one row of
    exact cancellation.  x: +1e-38, -1e-38, 1e-38 with every third negated,
    all zero.  w: the smallest subnormal everywhere; the same with the last
    product's sign flipped; then a zero product after the last nonzero one;
    alternating signs; all zero; +1.0 at k = 0 against -1.0 at k = 3;
    the first seven negative; -0 weights among positive tiny ones; past row
    7, all negative tiny."""
    x = np.full((4, k), np.float32(1e-38), np.float32)
    x[1] = -x[1]
    x[2, ::3] = -x[2, ::3]
    x[3] = 0
    w = np.full((max(n, 9), k), 0x0001, np.uint16)
    if k:
        w[1, k - 1] = 0x8001
        w[2, k - 1] = 0x0000
        w[3, 1::2] = 0x8001
        w[4] = 0
        w[5] = 0
        if k >= 4:  # x[0] and x[3] are equal in every activation row
            w[5, 0] = 0x3F80
            w[5, 3] = 0xBF80
        w[6, :7] = 0x8001
        w[7, ::5] = 0x8000
        w[8:] = 0x8001
    return x, np.ascontiguousarray(w[:n])


@pytest.mark.parametrize("n", [3, 8, 9])
@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("k", [1, 7, 1001, 4096, 4097, 8199, 14336])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_zero_outputs_follow_the_reference_chain(hip, k, m, n, layout):
    """A split-k sum that comes out exactly zero is settled by the reference's
    own chain (fmaf over ascending k from +0, jit.rs:29655-29670), so even the
    order-dependent zeros -- underflowing products whose sign changes along k,
    a +-0 product after the last nonzero one -- match bit for bit, through
    every FMA kernel: row-dot streaming, unaligned (odd K, short tails) and general,
    column-stream streaming (one slice or k split, odd N) and general (N = 3),
    one to four activation rows (four on K = 4096 / 14336 take the MFMA
    layout, which applies the same rule)."""
    x, w = zero_rows(k, n)
    x = np.ascontiguousarray(x[{1: [2], 2: [1, 2], 4: [0, 1, 2, 3]}[m]])
    y_ref = ref(x, w)
    assert np.all(y_ref == 0)
    y = RUN[layout](hip, x, w)
    bad = y.view(np.uint32) != y_ref.view(np.uint32)
    assert not bad.any(), (np.argwhere(bad)[:8], y[bad][:8], y_ref[bad][:8])


def test_zero_outputs_follow_the_reference_chain_batched_and_grouped(hip):
    """The zero rule through the batched column-stream entry (two slices, odd
    strides) and through a grouped row-dot launch of two problems."""
    k, n = 4104, 9
    x, w = zero_rows(k, n)
    xb = np.concatenate([x[2], np.zeros(3, np.float32), x[1]])       # ls = k + 3
    wt = np.ascontiguousarray(w.T).reshape(-1)
    wb = np.concatenate([wt, np.zeros(5, np.uint16), wt[::-1].copy()])  # rs = k*n + 5
    y = hip.matmul_bf16_gpu_batched(xb, wb, 1, k, n, 2, k + 3, k * n + 5)
    y_ref = oracle.matmul_bf16_batched(xb, wb, k, n, 2, k + 3, k * n + 5)
    assert np.array_equal(np.asarray(y).view(np.uint32), np.asarray(y_ref).view(np.uint32)), (y, y_ref)
    ws = [w, np.ascontiguousarray(w[::-1])]
    xs = [x[2:3].copy(), x[1:2].copy()]
    dxs = [hip.DeviceBuffer.from_numpy(v) for v in xs]
    dws = [hip.DeviceBuffer.from_numpy(v) for v in ws]
    dys = [hip.DeviceBuffer(4 * n) for _ in ws]
    try:
        hip.gemv_rd_grouped(dxs, dws, dys, [n, n], 1, k)
        hip.synchronize()
        for i in range(2):
            got = dys[i].download(np.float32, (n,))
            want = ref(xs[i], ws[i])[0]
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (i, got, want)
    finally:
        for b in dxs + dws + dys:
            b.free()


@pytest.mark.parametrize("k", [1, 7, 1000, 1001, 4096, 14336])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_underflowing_products_keep_their_zero_sign(hip, k, layout):
    """Row 0: every product is negative and underflows, so the reference chain
    (fmaf from +0.0, jit.rs:29655) ends at -0.0 -- and so does every other
    summation order, as long as the device's padding (lanes past K, windows
    past K, masked tails) adds only -0.0.  Row 1: the same products with the
    opposite sign end at +0.0.  (Products of both signs: see
    test_zero_outputs_follow_the_reference_chain.)"""
    x = np.full((1, k), np.float32(-1e-38), np.float32)
    w = np.full((2, k), 0x0001, np.uint16)     # smallest bf16 subnormal: |x*w| ~ 9e-79
    w[1, :] = 0x8001                           # row 1: positive products
    y_ref = ref(x, w)
    assert y_ref[0, 0] == 0 and np.signbit(y_ref[0, 0])
    assert y_ref[0, 1] == 0 and not np.signbit(y_ref[0, 1])
    y = RUN[layout](hip, x, w)
    check(y, y_ref, what=f"underflow signs k={k} {layout}")


@pytest.mark.parametrize("layout", LAYOUTS)
def test_k_zero_writes_positive_zero(hip, layout):
    x = np.zeros((2, 0), np.float32)
    w = np.zeros((5, 0), np.uint16)
    y = RUN[layout](hip, x, w)
    assert y.shape == (2, 5)
    assert np.all(y == 0) and not np.any(np.signbit(y))


def test_m_or_n_zero_leaves_out_untouched(hip):
    lib = hip._lib.load()
    out = np.full(4, 7.0, np.float32)
    x = np.ones(8, np.float32)
    w = np.ones(8, np.uint16)
    lib.dmc_matmul_bf16_gpu(x.ctypes.data, w.ctypes.data, out.ctypes.data, 0, 8, 4)
    lib.dmc_matmul_bf16_gpu(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, 8, 0)
    lib.dmc_matmul_bf16_gpu_batched(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, 8, 4, 0, 0, 0)
    assert np.all(out == 7.0)


# ---- the BASELINE configurations ---------------------------------------------------------

@pytest.mark.parametrize("layout", LAYOUTS)
def test_c1_full(hip, layout):
    w, x = W.c1()
    y = RUN[layout](hip, x, w)
    rel = check(y, ref(x, w), what=f"C1 {layout}")
    print(f"C1 {layout} rel={rel:.3e}")


@pytest.mark.parametrize("shape", W.C5_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("layout", LAYOUTS)
def test_c5_numerics(hip, shape, layout):
    n, k = shape
    w, x, rows = W.c5(n, k)
    y = RUN[layout](hip, x, w)[0]
    y_ref = ref(x, w)[0]
    rel = check(y, y_ref, what=f"C5 {shape} {layout}")
    print(f"C5 {shape} {layout} rel={rel:.3e}")
    # the rule each named row was built for (the oracle must agree, too)
    expect = {"inf_pos": "+inf", "inf_neg_x": "+inf", "inf_both": "nan", "inf_zero": "nan",
              "inf_nzero": "nan", "inf_tiny": "+inf", "inf_ntiny": "+inf", "nan_w": "nan",
              "zero_row": "+0", "negzero_row": "+0"}
    for name, cls in expect.items():
        for v in (y[rows[name]], y_ref[rows[name]]):
            if cls == "nan":
                assert np.isnan(v), (name, v)
            elif cls == "+inf":
                assert np.isposinf(v), (name, v)
            else:
                assert v == 0 and not np.signbit(v), (name, v)
    # all-subnormal weights: not flushed (nonzero, same sign), and within the
    # rigorous forward-error bound of two length-K fma chains, 2*K*u*sum|x*w|
    s = rows["sub_row"]
    terms = np.abs(x[0].astype(np.float64) * W.bf16_to_f32(w[s]).astype(np.float64))
    bound = 2 * k * 2.0 ** -24 * terms.sum()
    assert y_ref[s] != 0 and y[s] != 0 and np.signbit(y[s]) == np.signbit(y_ref[s]), (y[s], y_ref[s])
    assert abs(float(y[s]) - float(y_ref[s])) <= bound, (y[s], y_ref[s], bound)


@pytest.mark.parametrize("which", ["up", "down"])
def test_c2_sampled_rows(hip, which):
    """Full Llama-3-8B FFN shapes through the device-pointer entries; the
    oracle checks 512 random rows plus the first and last."""
    w, x = W.c2()[which]
    n, k = w.shape
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * n) as dy:
        hip.gemv_rd(dx, dw, dy, 1, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (n,))
    rng = np.random.default_rng(5)
    rows = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, 512)]))
    y_ref = oracle.gemv_points(x, w, "rd", np.zeros_like(rows), rows)
    rel = check(y[rows], y_ref, what=f"C2 {which}")
    print(f"C2 {which} rel={rel:.3e}")
    # the column-stream kernel on the transposed copy agrees as well
    wt = np.ascontiguousarray(w.T)
    with hip.DeviceBuffer.from_numpy(wt) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * n) as dy:
        hip.gemv_cs(dx, dw, dy, 1, k, n)
        hip.synchronize()
        y2 = dy.download(np.float32, (n,))
    check(y2[rows], y_ref, what=f"C2 {which} cs")


# (shape, m) -> rows16's plan: (blocks per workgroup, workgroups along N, k slices)
R16_C2_PLANS = {("down", 3): (2, 128, 2), ("down", 4): (2, 128, 2), ("down", 6): (2, 128, 2),
                ("down", 8): (2, 128, 2), ("down", 9): (4, 64, 4), ("down", 12): (4, 64, 4),
                ("down", 16): (4, 64, 4), ("up", 12): (4, 224, 1), ("up", 16): (4, 224, 1),
                ("down", 24): (4, 64, 2)}  # forced onto rows16: two activation tiles, each k-split


@pytest.mark.parametrize("shape,m", list(R16_C2_PLANS))
def test_rows16_split_k_on_c2(hip, shape, m, monkeypatch):
    """C2 at 3..16 activation rows on rows16.  Down (256 16-row blocks) keeps
    two blocks per workgroup at 3..8 rows and splits k in two, four blocks at
    9..16 rows and four k slices (256 workgroups either way), the slices summed
    by a second launch that settles zeros; up/gate at 12 and 16 rows runs four
    blocks per workgroup (224 workgroups) and k in one slice; down at 24 rows
    forced onto rows16 has two 16-row activation tiles, each on two k slices.  Activation row 1 is -1e-38
    throughout, so against the tiny weights planted in rows 0..3 (and the zero
    row 4) every product underflows: exact zeros whose signs follow the chain.
    Sampled rows (every block position, the planted ones, the last) against
    the oracle, within the norm and the elementwise bound."""
    w, x1 = W.c2()[shape]
    w = w.copy()
    n, k = w.shape
    rng = np.random.default_rng(40 + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0] = x1
    x[1] = np.float32(-1e-38)
    zrows = [1] + ([17] if m > 17 else [])  # one in each activation tile
    x[zrows] = np.float32(-1e-38)
    w[0:2] = 0x0001
    w[2:4] = 0x8001
    w[4] = 0
    w[5, : k // 2] = 0x3F80   # +1 then -1 against row 1's constant x: a cancellation
    w[5, k // 2:] = 0xBF80
    tiles, grid_x, ks = R16_C2_PLANS[(shape, m)]
    # rows16 named: the default above 16 rows is the gemm layout, and at 3
    # rows on down the 14-wave streaming kernel
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "7")
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * m * n) as dy:
        p = hip.plan("rd", m, k, n, x_addr=dx.addr, w_addr=dw.addr)
        assert (p.slices, p.rows_per_group, p.grid_x, p.workspace_bytes) == \
            (-7, 16 * tiles, grid_x, (ks * m * n * 4) if ks > 1 else 0), p
        hip.gemv_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (m, n))
    rows = np.unique(np.r_[np.arange(0, 40), np.arange(n - 20, n), rng.integers(0, n, 300)])
    mi, ni = np.meshgrid(np.arange(m), rows, indexing="ij")
    y_ref = oracle.gemv_points(x, w, "rd", mi.reshape(-1), ni.reshape(-1)).reshape(m, -1)
    check(y[:, rows], y_ref, what=f"rows16 C2 {shape} m={m}")
    for zr in zrows:
        assert np.all(y_ref[zr, :5] == 0)  # row 5 keeps a subnormal residue in the chain's order
        assert np.array_equal(y[zr, :5].view(np.uint32), y_ref[zr, :5].view(np.uint32)), \
            (zr, y[zr, :5], y_ref[zr, :5])
    wf = W.bf16_to_f32(w[rows])
    for r in range(m):
        check_bound(y[r, rows], y_ref[r], x[r], wf, what=f"rows16 C2 {shape} m={m} row {r}")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("layout", LAYOUTS)
def test_skinny_m(hip, m, layout):
    """The LM-head skinny batch on a 16,387-row slice of the C4 weight shape."""
    x, w = case(m, 4096, 16387, seed=77 + m, scale=0.02)
    y = RUN[layout](hip, x, w)
    check(y, ref(x, w), what=f"skinny m={m} {layout}")


# ---- batched / deferred protocol (gpu.rs:410-474) ----------------------------------------

def test_batched_matches_per_slice(hip):
    k, n, batch = 256, 64, 6
    ls, rs = k + 8, k * n + 64
    rng = np.random.default_rng(3)
    x = rng.standard_normal((batch - 1) * ls + k).astype(np.float32)
    w = W.bf16_rne(rng.standard_normal((batch - 1) * rs + k * n).astype(np.float32))
    y = hip.matmul_bf16_gpu_batched(x, w, 1, k, n, batch, ls, rs)
    y_ref = oracle.matmul_bf16_batched(x, w, k, n, batch, ls, rs)
    check(y, y_ref, what="batched")


def test_batched_broadcast_activation(hip):
    # ls = 0: every slice reads the same activation (the broadcast [B,1,S,K] case)
    k, n, batch = 128, 32, 9
    rng = np.random.default_rng(4)
    x = rng.standard_normal(k).astype(np.float32)
    w = W.bf16_rne(rng.standard_normal(batch * k * n).astype(np.float32))
    y = hip.matmul_bf16_gpu_batched(x, w, 1, k, n, batch, 0, k * n)
    check(y, oracle.matmul_bf16_batched(x, w, k, n, batch, 0, k * n), what="broadcast")


@pytest.mark.parametrize("batch,k,n", [(8, 4096, 128), (32, 4096, 128), (3, 1001, 77), (5, 64, 1)])
def test_batched_broadcast_stacked_rowdot(hip, batch, k, n, monkeypatch):
    """Slices that share one activation row over weights one after another
    (per-head projections of one token: ls = 0, m = 1, rs = k n) run as one
    row-dot GEMV over the slices' stacked transposes, resident after the
    first call; the same calls on the column-stream kernels
    (DMC_HIP_CS_LAYOUT=1) and the oracle agree.  Special weights included;
    the deferred protocol too."""
    rng = np.random.default_rng(batch * 7 + k + n)
    x = rng.standard_normal(k).astype(np.float32)
    x[::17] = 0.0
    w = W.bf16_rne(np.float32(0.02) * rng.standard_normal(batch * k * n).astype(np.float32))
    pos = rng.integers(0, w.size, size=max(1, w.size // 500))
    w[pos] = rng.choice(np.array([0x0001, 0x8001, 0x0000, 0x8000, 0x7F80, 0xFF80], np.uint16), size=pos.size)
    y_ref = oracle.matmul_bf16_batched(x, w, k, n, batch, 0, k * n)
    for _ in range(2):  # upload and transpose, then the resident copy
        y = hip.matmul_bf16_gpu_batched(x, w, 1, k, n, batch, 0, k * n)
        check(y, y_ref, what=f"stacked row-dot batch={batch} k={k} n={n}")
    out = np.full(batch * n, np.nan, np.float32)
    hip.matmul_bf16_gpu_batched_deferred(x, w, out, 1, k, n, batch, 0, k * n)
    hip.flush()
    check(out, y_ref, what="stacked row-dot, deferred")
    monkeypatch.setenv("DMC_HIP_CS_LAYOUT", "1")
    check(hip.matmul_bf16_gpu_batched(x, w, 1, k, n, batch, 0, k * n), y_ref, what="column-stream layout")


def test_deferred_then_flush(hip):
    k, n = 512, 256
    rng = np.random.default_rng(6)
    outs, refs = [], []
    for i in range(5):
        x = rng.standard_normal(k).astype(np.float32)
        w = W.bf16_rne(rng.standard_normal(k * n).astype(np.float32))
        refs.append(oracle.matmul_bf16_batched(x, w, k, n, 1, 0, 0))
        out = np.full(n, np.nan, np.float32)
        hip.matmul_bf16_gpu_batched_deferred(x, w, out, 1, k, n, 1, 0, 0)
        x[:] = 12345.0  # inputs are copied before return; this must not leak in
        outs.append(out)
    hip.flush()
    for out, y_ref in zip(outs, refs):
        check(out, y_ref, what="deferred")


def test_sync_call_materializes_deferred(hip):
    k, n = 256, 128
    rng = np.random.default_rng(8)
    x1 = rng.standard_normal(k).astype(np.float32)
    w1 = W.bf16_rne(rng.standard_normal(k * n).astype(np.float32))
    out1 = np.full(n, np.nan, np.float32)
    hip.matmul_bf16_gpu_batched_deferred(x1, w1, out1, 1, k, n, 1, 0, 0)
    x2 = rng.standard_normal((1, k)).astype(np.float32)
    w2 = W.bf16_rne(rng.standard_normal((k, n)).astype(np.float32))
    y2 = hip.matmul_bf16_gpu(x2, w2)
    check(out1, oracle.matmul_bf16_batched(x1, w1, k, n, 1, 0, 0), what="deferred by sync")
    check(y2, oracle.matmul_bf16(x2, w2), what="sync")


def test_overlap_with_pending_output_flushes_first(hip):
    # the second call reads the first call's pending output as its activation
    k = n = 128
    rng = np.random.default_rng(9)
    x = rng.standard_normal(k).astype(np.float32)
    w = W.bf16_rne(rng.standard_normal(k * n).astype(np.float32))
    mid = np.full(n, np.nan, np.float32)
    hip.matmul_bf16_gpu_batched_deferred(x, w, mid, 1, k, n, 1, 0, 0)
    out = np.empty(n, np.float32)
    hip.matmul_bf16_gpu_batched_deferred(mid, w, out, 1, k, n, 1, 0, 0)
    hip.flush()
    ref_mid = oracle.matmul_bf16_batched(x, w, k, n, 1, 0, 0)
    check(mid, ref_mid, what="first")
    check(out, oracle.matmul_bf16_batched(ref_mid, w, k, n, 1, 0, 0), tol=1e-4, what="chained")


# ---- residency and determinism -----------------------------------------------------------

def test_weights_resident_by_content(hip):
    hip.release_weights()
    x, w = case(1, 1024, 512, seed=11)
    wt = np.ascontiguousarray(w.T)
    y1 = hip.matmul_bf16_gpu(x, wt)
    assert hip.resident_count() == 1
    wt_copy = wt.copy()                       # same bytes, new address: no upload
    y2 = hip.matmul_bf16_gpu(x, wt_copy)
    assert hip.resident_count() == 1
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    wt_copy[0, 0] ^= 1                        # one sampled word differs: new entry
    hip.matmul_bf16_gpu(x, wt_copy)
    assert hip.resident_count() == 2
    hip.release_weights()
    assert hip.resident_count() == 0 and hip.resident_bytes() == 0


def test_register_weight_then_call(hip):
    """A registered weight keeps the caller's layout: the x @ W' entry and the
    batched x @ W entry (column-stream kernels) reuse it without an upload."""
    hip.release_weights()
    x, w = case(1, 2048, 300, seed=12)
    assert hip.register_weight(w) != 0
    assert hip.resident_count() == 1
    y = hip.matmul_bf16_gpu_t(x, w)
    assert hip.resident_count() == 1
    check(y, ref(x, w), what="registered rd")
    wt = np.ascontiguousarray(w.T)
    assert hip.register_weight(wt) != 0
    assert hip.resident_count() == 2
    xb = np.concatenate([x[0], x[0]])
    y2 = hip.matmul_bf16_gpu_batched(xb, wt, 1, 2048, 300, 2, 2048, 0)
    assert hip.resident_count() == 2
    check(y2[:300], ref(x, w)[0], what="registered batched cs")
    check(y2[300:], ref(x, w)[0], what="registered batched cs, slice 1")


def test_dropin_x_at_w_keeps_one_transposed_copy(hip, monkeypatch):
    """A single-slice x @ W uploads W once, transposed for the row-dot
    kernels, and reuses that copy; DMC_HIP_CS_LAYOUT=1 runs the
    column-stream kernels on the weight as given instead.  Both match."""
    hip.release_weights()
    x, w = case(2, 3000, 777, seed=14, edge=True)
    wt = np.ascontiguousarray(w.T)
    y1 = hip.matmul_bf16_gpu(x, wt)
    assert hip.resident_count() == 1 and hip.resident_bytes() == wt.nbytes
    y2 = hip.matmul_bf16_gpu(x, wt.copy())
    assert hip.resident_count() == 1
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    monkeypatch.setenv("DMC_HIP_CS_LAYOUT", "1")
    y3 = hip.matmul_bf16_gpu(x, wt)
    assert hip.resident_count() == 2           # the as-given copy
    y_ref = ref(x, w)
    check(y1, y_ref, what="x@W transposed copy")
    check(y3, y_ref, what="x@W column-stream")
    hip.release_weights()


@pytest.mark.parametrize("layout", LAYOUTS)
def test_repeat_calls_bit_identical(hip, layout):
    x, w = case(1, 14336, 1024, seed=13, scale=0.02)
    run = RUN[layout]
    a = run(hip, x, w)
    b = run(hip, x, w)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- column-stream split-K finish (last workgroup sums the slices) ----------------------

@pytest.mark.parametrize("m,k,n,batch", [(1, 3000, 1032, 1), (9, 3000, 1032, 1), (1, 2048, 520, 40),
                                         (3, 14336, 4096, 1), (2, 777, 8, 5)])
def test_cs_split_k_counters_reset(hip, m, k, n, batch):
    """Several calls in a row through the split-K streaming kernel: each must
    match the oracle and repeat bit for bit (the slice counters return to zero
    after every launch; a stale counter would finish a column block early)."""
    rng = np.random.default_rng(m * 131 + k + n + batch)
    ls, rs = m * k, k * n
    x = rng.standard_normal(batch * m * k).astype(np.float32)
    w = W.bf16_rne(np.float32(0.05) * rng.standard_normal(batch * k * n).astype(np.float32))
    plan = hip.plan("cs", m, k, n, batch=batch, rs=rs, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert plan.vec == 8 and plan.waves > 0
    if k >= 2048:
        assert plan.slices > 1, plan
    ref_parts = []
    for z in range(batch):
        ref_parts.append(oracle.matmul_bf16(x[z * ls:(z + 1) * ls].reshape(m, k),
                                            w[z * rs:(z + 1) * rs].reshape(k, n)).reshape(-1))
    y_ref = np.concatenate(ref_parts)
    first = None
    for _ in range(3):
        y = hip.matmul_bf16_gpu_batched(x, w, m, k, n, batch, ls, rs)
        check(y, y_ref, what=f"cs split-K m={m} k={k} n={n} batch={batch}")
        if first is None:
            first = y.copy()
        assert np.array_equal(y.view(np.uint32), first.view(np.uint32))


# ---- grouped row-dot launch and the device weight generator ------------------------------

@pytest.mark.parametrize("k,ns,m", [(4096, [4096, 1024, 1024], 1), (14336, [4096, 520], 2),
                                    (4097, [300, 7], 1), (1000, [64, 0, 33], 3),
                                    (512, [1, 2, 3, 4, 5, 6, 7, 8, 9, 10], 1)])
def test_grouped_rowdot_matches_each_problem(hip, k, ns, m):
    """Independent problems sharing x's shape in one launch (q/k/v, gate/up):
    each output equals its own GEMV's reference; more than 8 problems and
    shapes outside the streaming kernel take the per-launch path."""
    rng = np.random.default_rng(k + len(ns) * 7 + m)
    xs, ws = [], []
    for i, n in enumerate(ns):
        xs.append(rng.standard_normal((m, k)).astype(np.float32))
        ws.append(W.bf16_rne(np.float32(0.02) * rng.standard_normal((n, k)).astype(np.float32)))
    dxs = [hip.DeviceBuffer.from_numpy(x) for x in xs]
    dws = [hip.DeviceBuffer.from_numpy(w) if w.size else hip.DeviceBuffer(16) for w in ws]
    dys = [hip.DeviceBuffer(max(4 * m * n, 4)) for n in ns]
    try:
        hip.gemv_rd_grouped(dxs, dws, dys, ns, m, k)
        hip.synchronize()
        got, want = [], []
        for i, n in enumerate(ns):
            if n == 0:
                continue
            y = dys[i].download(np.float32, (m, n))
            rows = np.arange(n) if n <= 1100 else np.unique(np.r_[0, n - 1, rng.integers(0, n, 300)])
            mi, ni = np.meshgrid(np.arange(m), rows, indexing="ij")
            y_ref = oracle.gemv_points(xs[i], ws[i], "rd", mi.reshape(-1), ni.reshape(-1))
            yd = y[:, rows].reshape(-1)
            wf = W.bf16_to_f32(ws[i][rows])
            for r in range(m):
                check_bound(y[r, rows], y_ref.reshape(m, -1)[r], xs[i][r], wf, what=f"grouped problem {i}")
            if n >= 256:
                check(yd, y_ref, what=f"grouped k={k} problem {i} n={n}")
            got.append(yd)
            want.append(y_ref)
        # the normwise rule over the whole group (a one-output problem alone is
        # ill-conditioned for a norm)
        check(np.concatenate(got), np.concatenate(want), what=f"grouped k={k} all problems")
    finally:
        for b in dxs + dws + dys:
            b.free()


def test_device_fill_matches_host_generator(hip):
    table = W.normal_table(0.02)
    n, off = 1_000_003, 123_457
    key = W.counter_seed(0, 5)
    with hip.DeviceBuffer.from_numpy(table) as dt, hip.DeviceBuffer(2 * n) as dst:
        hip.fill_counter_bf16(dst, n, key, dt, offset=off)
        hip.synchronize()
        got = dst.download(np.uint16, (n,))
    assert np.array_equal(got, W.counter_bf16(0, 5, n, offset=off))


def test_graph_replay_matches_oracle_each_time(hip):
    """A captured step (one GEMV and one grouped pair) replayed three times,
    with new activations uploaded eagerly between replays: every replay must
    read the live inputs and match the reference."""
    k = 4096
    rng = np.random.default_rng(21)
    ns = [1000, 300, 520]
    ws = [W.bf16_rne(np.float32(0.02) * rng.standard_normal((n, k)).astype(np.float32)) for n in ns]
    dws = [hip.DeviceBuffer.from_numpy(w) for w in ws]
    dx = hip.DeviceBuffer(4 * k)
    dys = [hip.DeviceBuffer(4 * n) for n in ns]
    try:
        dx.upload(rng.standard_normal(k).astype(np.float32))
        hip.gemv_rd(dx, dws[0], dys[0], 1, k, ns[0])          # eager warm-up of the same shapes
        hip.gemv_rd_grouped([dx, dx], dws[1:], dys[1:], ns[1:], 1, k)
        hip.synchronize()
        g = hip.Graph()
        with g:
            hip.gemv_rd(dx, dws[0], dys[0], 1, k, ns[0])
            hip.gemv_rd_grouped([dx, dx], dws[1:], dys[1:], ns[1:], 1, k)
        try:
            for rep in range(3):
                x = rng.standard_normal(k).astype(np.float32)
                dx.upload(x)
                for b, n in zip(dys, ns):
                    b.upload(np.full(n, np.nan, np.float32))
                g.launch()
                hip.synchronize()
                for i, n in enumerate(ns):
                    y = dys[i].download(np.float32, (n,))
                    check(y, oracle.matmul_bf16_t(x, ws[i])[0], what=f"graph replay {rep} problem {i}")
        finally:
            g.destroy()
    finally:
        for b in dws + dys + [dx]:
            b.free()


def test_graph_replay_after_workspace_growth(hip, monkeypatch):
    """A graph captured around a gemm-layout GEMV (its x planes and partial
    sums live in the library workspace), then a larger eager call that
    outgrows the workspace, then the graph replayed: the replay must still
    see a live workspace and match the reference, and so must eager calls
    after the graph is destroyed."""
    k, n, m1, m2 = 1024, 600, 24, 4096  # m2's workspace (~45 MB) outgrows every earlier test's
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "8")  # a matrix this small runs rows16 by default
    x1, w = case(m1, k, n, seed=4242, scale=0.02)
    x2, _ = case(m2, k, n, seed=4243, scale=0.02)
    dw = hip.DeviceBuffer.from_numpy(w)
    dx1, dx2 = hip.DeviceBuffer.from_numpy(x1), hip.DeviceBuffer.from_numpy(x2)
    dy1, dy2 = hip.DeviceBuffer(4 * m1 * n), hip.DeviceBuffer(4 * m2 * n)
    try:
        p1 = hip.plan("rd", m1, k, n, x_addr=256, w_addr=256)
        p2 = hip.plan("rd", m2, k, n, x_addr=256, w_addr=256)
        assert p1.slices == -8 and p2.workspace_bytes > 2 * p1.workspace_bytes, (p1, p2)
        hip.gemv_rd(dx1, dw, dy1, m1, k, n)                   # sizes the workspace for m1
        hip.synchronize()
        g = hip.Graph()
        with g:
            hip.gemv_rd(dx1, dw, dy1, m1, k, n)
        try:
            hip.gemv_rd(dx2, dw, dy2, m2, k, n)               # outgrows it
            hip.synchronize()
            sample = [0, 1, m2 // 2, m2 - 1]
            check(dy2.download(np.float32, (m2, n))[sample], ref(x2[sample], w), what="eager m2 after growth")
            for rep in range(2):
                dy1.upload(np.full(m1 * n, np.nan, np.float32))
                g.launch()
                hip.synchronize()
                check(dy1.download(np.float32, (m1, n)), ref(x1, w), what=f"replay {rep} after growth")
        finally:
            g.destroy()
        hip.gemv_rd(dx1, dw, dy1, m1, k, n)
        hip.synchronize()
        check(dy1.download(np.float32, (m1, n)), ref(x1, w), what="eager m1 after destroy")
    finally:
        for b in (dw, dx1, dx2, dy1, dy2):
            b.free()


def test_graph_replay_rows16_k_split(hip):
    """A rows16 plan that splits k (C2 down at m = 6: partial sums in the
    library workspace, then the slice-sum launch), captured after one
    uncaptured call of the same shape, replayed three times with new
    activations uploaded eagerly in between: every replay must match the
    reference (sampled rows, every activation row)."""
    n, k, m = 4096, 14336, 6
    p = hip.plan("rd", m, k, n, x_addr=256, w_addr=256)
    assert p.slices == -7 and p.workspace_bytes > 0, p
    rng = np.random.default_rng(77)
    w = W.bf16_rne(np.float32(0.02) * rng.standard_normal((n, k)).astype(np.float32))
    rows = np.unique(np.r_[0, n - 1, rng.integers(0, n, 96), np.arange(15, n, 512)])
    dw, dx, dy = hip.DeviceBuffer.from_numpy(w), hip.DeviceBuffer(4 * m * k), hip.DeviceBuffer(4 * m * n)
    try:
        dx.upload(rng.standard_normal((m, k)).astype(np.float32))
        hip.gemv_rd(dx, dw, dy, m, k, n)  # sizes the workspace for this shape
        hip.synchronize()
        g = hip.Graph()
        with g:
            hip.gemv_rd(dx, dw, dy, m, k, n)
        try:
            for rep in range(3):
                x = rng.standard_normal((m, k)).astype(np.float32)
                dx.upload(x)
                dy.upload(np.full(m * n, np.nan, np.float32))
                g.launch()
                hip.synchronize()
                y = dy.download(np.float32, (m, n))
                check(y[:, rows], ref(x, w[rows]), what=f"rows16 k-split replay {rep}")
        finally:
            g.destroy()
    finally:
        for b in (dw, dx, dy):
            b.free()


def test_c3_layer_schedule(hip):
    """One layer of the C3 decode sweep as the bench runs it: weights filled in
    HBM by the counter generator, q/k/v and gate/up as grouped launches, o and
    down single, all captured in a graph; sampled rows of every projection
    against the reference on host-regenerated rows."""
    layer = 7
    names = [nm for nm, _, _ in W.LLAMA3_8B_LAYER]
    shape = {nm: (n, k) for nm, n, k in W.LLAMA3_8B_LAYER}
    table = hip.DeviceBuffer.from_numpy(W.normal_table(W.C3_SCALE))
    ws = {nm: hip.DeviceBuffer(2 * shape[nm][0] * shape[nm][1]) for nm in names}
    x, x2 = W.c3_x(layer, 4096), W.c3_x(layer, 14336)
    dx, dx2 = hip.DeviceBuffer.from_numpy(x), hip.DeviceBuffer.from_numpy(x2)
    ys = {nm: hip.DeviceBuffer(4 * shape[nm][0]) for nm in names}
    try:
        for idx, nm in enumerate(names):
            n, k = shape[nm]
            hip.fill_counter_bf16(ws[nm], n * k, W.counter_seed(0, W.c3_tensor(layer, idx)), table)

        def step():
            hip.gemv_rd_grouped([dx] * 3, [ws["q"], ws["k"], ws["v"]], [ys["q"], ys["k"], ys["v"]],
                                [4096, 1024, 1024], 1, 4096)
            hip.gemv_rd(dx, ws["o"], ys["o"], 1, 4096, 4096)
            hip.gemv_rd_grouped([dx] * 2, [ws["gate"], ws["up"]], [ys["gate"], ys["up"]], [14336] * 2, 1, 4096)
            hip.gemv_rd(dx2, ws["down"], ys["down"], 1, 14336, 4096)

        step()
        hip.synchronize()
        g = hip.Graph()
        with g:
            step()
        try:
            for b in ys.values():
                b.upload(np.full(b.nbytes // 4, np.nan, np.float32))
            g.launch()
            hip.synchronize()
        finally:
            g.destroy()
        rng = np.random.default_rng(layer)
        for idx, nm in enumerate(names):
            n, k = shape[nm]
            rows = np.unique(np.r_[0, n - 1, rng.integers(0, n, 40)])
            wr = W.c3_rows(layer, idx, rows)
            xv = x2 if nm == "down" else x
            y_ref = oracle.matmul_bf16_t(xv, wr)[0]
            y = ys[nm].download(np.float32, (n,))
            check(y[rows], y_ref, what=f"C3 layer {layer} {nm}")
    finally:
        for b in list(ws.values()) + list(ys.values()) + [dx, dx2, table]:
            b.free()


# ---- skinny M on MFMA: special values through the three-term split ---------------------

@pytest.mark.parametrize("kind", [6, 7, 8])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 8, 16, 20])
def test_skinny_mfma_special_values(hip, m, kind, monkeypatch):
    """The MFMA path (M >= 2) against the reference chain on data full of
    special values: bf16 subnormal weights, +-inf / NaN weights, +-0 and
    f32-subnormal activations, an infinite and a NaN activation, the smallest
    subnormals (whose bf16 truncation is 0), and an all-zero weight row."""
    k, n = 1024, 333
    x, w = case(m, k, n, seed=900 + m, edge=True)
    x[0, 5] = np.inf
    x[1, 7] = np.nan
    if m >= 4:
        x[2, 9] = np.float32(1.4e-45)      # 2^-149
        x[3, 11] = np.float32(-1.4e-45)
    w[10, 9] = 0x7F80                  # +inf against 2^-149: +inf (not NaN)
    w[11, 11] = 0xFF80                 # -inf against -2^-149: +inf
    w[12, :] = 0                       # exact zero products: +0
    w[13, 100] = 0x7F80                # +inf against a normal x in every row
    w[14, 200] = 0x7FC1                # NaN
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", str(kind))
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "2")  # M = 2 included
    p = hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert p.slices == -kind, "expected the MFMA kernel"
    y = run_rd(hip, x, w)
    y_ref = ref(x, w)
    check(y, y_ref, what=f"mfma specials m={m}")
    if m >= 4:
        assert np.isposinf(y_ref[2, 10]) and np.isposinf(y[2, 10])
        assert np.isposinf(y_ref[3, 11]) and np.isposinf(y[3, 11])
    assert np.all(y[:, 12][np.isfinite(y_ref[:, 12])] == 0)


@pytest.mark.parametrize("kind", [6, 7, 8])
@pytest.mark.parametrize("m,k,n", [(4, 4096, 16387), (16, 14336, 4096), (8, 64, 70), (5, 11008, 1000),
                                   (16, 4096, 40000), (3, 320, 300), (2, 4096, 16387), (2, 64, 70),
                                   (4, 14336, 1001), (7, 576, 33), (12, 128, 17)])
def test_skinny_mfma_shapes_within_bound(hip, m, k, n, kind, monkeypatch):
    """MFMA tiles, k split over waves or chunked through LDS, partial tiles
    and chunks: every element within the rigorous forward-error bound of the
    reference chain."""
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", str(kind))
    monkeypatch.setenv("DMC_HIP_RD_MFMA_MIN_M", "2")  # M = 2 included
    x, w = case(m, k, n, seed=m + k + n, scale=0.02)
    assert hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data).slices == -kind
    y = run_rd(hip, x, w)
    rows = np.unique(np.r_[0, n - 1, np.random.default_rng(1).integers(0, n, 200)])
    y_ref = oracle.matmul_bf16_t(x, w[rows])
    wf = W.bf16_to_f32(w[rows])
    for r in range(m):
        check_bound(y[r, rows], y_ref[r], x[r], wf, what=f"mfma m={m} k={k} n={n} row {r}")
    check(y[:, rows], y_ref, what=f"mfma m={m} k={k} n={n}")


# ---- row-dot streaming with x shared through LDS (16-wave workgroups, M = 1) ----------

XLDS_SHAPES = [(4096, 14336), (4096, 4112), (8192, 8192), (4096, 16384), (16380, 12288)]


@pytest.mark.parametrize("n,k", XLDS_SHAPES)
def test_shared_x_workgroups(hip, n, k, monkeypatch):
    """Long rows at M = 1 on 16-wave workgroups whose halves share one LDS
    copy of x (the layout for K above 14336; DMC_HIP_RD_X14=0 keeps it for
    shorter rows): a last block of two windows (k = 4112), the largest K it
    takes, two rounds (n = 8192), and a partial last workgroup whose second
    half holds 4 rows (n = 16380, four rounds)."""
    monkeypatch.setenv("DMC_HIP_RD_XLDS", "1")
    monkeypatch.setenv("DMC_HIP_RD_X14", "0")
    assert hip.plan("rd", 1, k, n).waves == 16
    x, w = case(1, k, n, seed=7000 + n + k, edge=True)
    check(run_rd(hip, x, w), ref(x, w), what=f"xlds n={n} k={k}")


@pytest.mark.parametrize("k", [4112, 14336])
def test_shared_x_zero_signs(hip, k, monkeypatch):
    """The zero-sign rule of test_underflowing_products_keep_their_zero_sign on
    the shared-x layout: even rows end at -0.0, odd rows at +0.0."""
    monkeypatch.setenv("DMC_HIP_RD_XLDS", "1")
    monkeypatch.setenv("DMC_HIP_RD_X14", "0")
    n = 4096
    assert hip.plan("rd", 1, k, n).waves == 16
    x = np.full((1, k), np.float32(-1e-38), np.float32)
    w = np.full((n, k), 0x0001, np.uint16)
    w[1::2, :] = 0x8001
    y_ref = ref(x, w)
    assert np.all(np.signbit(y_ref[0, 0::2])) and not np.any(np.signbit(y_ref[0, 1::2]))
    check(run_rd(hip, x, w), y_ref, what=f"xlds zero signs k={k}")
    # products of both signs (order-dependent zeros), every pattern of
    # zero_rows in turn over the 4096 rows, against x with mixed signs
    xm, wz = zero_rows(k, 9)
    w = np.ascontiguousarray(wz[np.arange(n) % 9])
    xm = np.ascontiguousarray(xm[2:3])
    y_ref = ref(xm, w)
    y = run_rd(hip, xm, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))[:8]


@pytest.mark.parametrize("n,k", [(1030, 4096), (1, 4096), (4097, 4000), (2049, 2048), (7, 1024), (8190, 4096)])
def test_four_rows_per_step_on_small_grids(hip, n, k, monkeypatch):
    """One activation row, one window per lane and at most 8 four-row
    workgroups per CU: 4 rows in one step, 4 per workgroup (partial last
    workgroups: n = 1030, 4097, 2049, 7; a lone row; fewer waves at k = 2048
    and 1024; n = 8190 with the 8-wave group switched off).  Edge data; the
    parity rule and, row by row, the bound; the zero rule's rare path on rows
    of underflowing products."""
    monkeypatch.setenv("DMC_HIP_RD_X8", "0")
    p = hip.plan("rd", 1, k, n, x_addr=256, w_addr=256)
    assert (p.rows_or_rw, p.rows_per_group) == (4, 4), p
    x, w = case(1, k, n, seed=7300 + n + k, edge=True)
    check_or_bound(run_rd(hip, x, w), ref(x, w), x, W.bf16_to_f32(w), what=f"4 rows per step n={n} k={k}")
    xz = np.full((1, k), np.float32(-1e-38), np.float32)
    wz = np.full((n, k), 0x0001, np.uint16)
    wz[1::2] = 0x8001
    y_ref = ref(xz, wz)
    y = run_rd(hip, xz, wz)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))


X14_SHAPES = [(4096, 14336), (4097, 14336), (8190, 12288), (4096, 4112), (1030, 14336), (6, 9000), (16384, 12288)]


def _rd_dev(hip, x, w, y_init=np.nan):
    m, k = x.shape
    n = w.shape[0]
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * m * n) as dy:
        dy.upload(np.full(m * n, y_init, np.float32))
        hip.gemv_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        return dy.download(np.float32, (m, n))


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", X14_SHAPES)
def test_shared_x_fourteen_waves(hip, n, k, m, monkeypatch):
    """One group of 14 waves splitting k (the default for 4096 < K <= 14336
    at M = 1 to 4; DMC_HIP_RD_XLDS=2 takes it wherever it applies), with one
    to four activation rows (x in registers): C2 down (two windows per lane,
    all carrying data), a partial last workgroup (n = 4097: one row of 16),
    one window per lane (k = 4112, its last block holding 16 elements),
    fewer rows than one workgroup (n = 6), and 1024 workgroups.  Edge data;
    the oracle's result within the parity rule and, row by row, the
    elementwise bound; two launches bit for bit alike."""
    x, w = case(m, k, n, seed=7100 + n + k + m, edge=True)
    monkeypatch.setenv("DMC_HIP_RD_XLDS", "2")
    p = hip.plan("rd", m, k, n, x_addr=256, w_addr=256)
    assert (p.waves, p.rows_per_group, p.slices, p.mt) == (14, 16, 1 if k <= 7168 else 2, m), p
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), _rd_dev(hip, x, w).view(np.uint32))
    check_or_bound(y, ref(x, w), x, W.bf16_to_f32(w), what=f"x14 m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [4112, 14336])
def test_shared_x_fourteen_waves_zero_rule(hip, k, m, monkeypatch):
    """Exact zeros on the 14-wave kernel, one to four activation rows:
    underflowing products of one sign (zero signs from the chain) and the
    rows of zero_rows' patterns (order-dependent zeros, exact-zero products)
    -- bit for bit the reference."""
    monkeypatch.setenv("DMC_HIP_RD_XLDS", "2")
    n = 4096
    assert hip.plan("rd", m, k, n, x_addr=256, w_addr=256).waves == 14
    x = np.full((m, k), np.float32(-1e-38), np.float32)
    x[1::2] = -x[1::2]                       # odd rows: the opposite zero signs
    w = np.full((n, k), 0x0001, np.uint16)
    w[1::2, :] = 0x8001
    y_ref = ref(x, w)
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    xm, wz = zero_rows(k, 9)
    w = np.ascontiguousarray(wz[np.arange(n) % 9])
    xm = np.ascontiguousarray(xm[(2 + np.arange(m)) % 4])
    y_ref = ref(xm, w)
    y = _rd_dev(hip, xm, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), \
        np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))[:8]


X8_SHAPES = [(14336, 4096), (4097, 4096), (1030, 4000), (6, 3000), (1, 4096), (1792, 4096), (16384, 2056)]
PER_CU_ROWS = (4, 6, 7, 8, 10, 12, 14)


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", X8_SHAPES)
def test_eight_wave_group(hip, n, k, m, monkeypatch):
    """The 14-wave kernel's layout on one group of 8 waves (K <= 4096: one
    window per lane, x in registers), forced with DMC_HIP_RD_X8=2: C2
    up/gate, a partial last workgroup (n = 4097), lanes past K (k = 4000,
    3000, 2056), fewer rows than one workgroup (n = 6, a lone row), a TP = 8
    share, 1024 workgroups.  Edge data; the oracle's result within the
    parity rule and, row by row, the elementwise bound; two launches bit for
    bit alike."""
    x, w = case(m, k, n, seed=7700 + n + k + m, edge=True)
    monkeypatch.setenv("DMC_HIP_RD_X8", "2")
    p = hip.plan("rd", m, k, n, x_addr=256, w_addr=256)
    rpc = n // 256 if n % 256 == 0 and n // 256 in PER_CU_ROWS and (m == 1 or n // 256 <= 12) else 0  # per CU
    want = (8, rpc if rpc <= 8 else rpc // 2, rpc, 1, m, 256) if rpc else (8, 4, 16, 1, m, -(-n // 16))
    assert (p.waves, p.rows_or_rw, p.rows_per_group, p.slices, p.mt, p.grid_x) == want, p
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), _rd_dev(hip, x, w).view(np.uint32))
    check_or_bound(y, ref(x, w), x, W.bf16_to_f32(w), what=f"x8 m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [4096, 2056])
def test_eight_wave_group_zero_rule(hip, k, m, monkeypatch):
    """Exact zeros on the 8-wave group, one to four activation rows: the
    patterns of test_shared_x_fourteen_waves_zero_rule, bit for bit the
    reference."""
    monkeypatch.setenv("DMC_HIP_RD_X8", "2")
    n = 4096
    assert hip.plan("rd", m, k, n, x_addr=256, w_addr=256).waves == 8
    x = np.full((m, k), np.float32(-1e-38), np.float32)
    x[1::2] = -x[1::2]
    w = np.full((n, k), 0x0001, np.uint16)
    w[1::2, :] = 0x8001
    y_ref = ref(x, w)
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    xm, wz = zero_rows(k, 9)
    w = np.ascontiguousarray(wz[np.arange(n) % 9])
    xm = np.ascontiguousarray(xm[(2 + np.arange(m)) % 4])
    y_ref = ref(xm, w)
    y = _rd_dev(hip, xm, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), \
        np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))[:8]


PER_CU_CASES = [(n, k, m) for (n, k) in [(1024, 4096), (1536, 4096), (1792, 4096), (2048, 4000), (2560, 4096),
                                         (3072, 3000), (3584, 4096), (1792, 2056)]
                for m in (1, 2, 3, 4) if m == 1 or n // 256 <= 12]


@pytest.mark.parametrize("n,k,m", PER_CU_CASES)
def test_one_group_per_cu(hip, n, k, m):
    """N = r * 256 rows (r = 4 .. 14): one 8-wave group of r rows per CU, the
    planner's own choice at one activation row (the drop-in's stacked k/v
    heads, TP = 8's gate/up share) and at two to four up to r = 12, with
    lanes past K (k = 4000, 3000, 2056).  Edge data within the parity rule
    and, row by row, the bound; the zero rule's patterns bit for bit the
    reference."""
    r = n // 256
    p = hip.plan("rd", m, k, n, x_addr=256, w_addr=256)
    assert (p.waves, p.rows_or_rw, p.rows_per_group, p.mt, p.grid_x) == (8, r if r <= 8 else r // 2, r, m, 256), p
    x, w = case(m, k, n, seed=7800 + n + k + m, edge=True)
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), _rd_dev(hip, x, w).view(np.uint32))
    check_or_bound(y, ref(x, w), x, W.bf16_to_f32(w), what=f"group per CU m={m} n={n} k={k}")
    xm, wz = zero_rows(k, 9)
    wz = np.ascontiguousarray(wz[np.arange(n) % 9])
    xm = np.ascontiguousarray(xm[(np.arange(m) + (m - 1)) % 4]) if m > 1 else None
    for row in range(4) if m == 1 else [None]:
        xr = np.ascontiguousarray(xm if m > 1 else zero_rows(k, 9)[0][row:row + 1])
        y_ref = ref(xr, wz)
        y = _rd_dev(hip, xr, wz)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), \
            (row, np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))[:8])


X4_SHAPES = [(4096, 1792), (4097, 2048), (1030, 1000), (6, 1504), (1, 2048), (8192, 2048), (300, 64)]


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("n,k", X4_SHAPES)
def test_four_wave_group(hip, n, k, m, monkeypatch):
    """The same group on 4 waves (K <= 2048), forced with DMC_HIP_RD_X8=2:
    TP = 8's down share, a partial last workgroup (n = 4097), lanes past K
    (k = 1792, 1000, 1504, 64), fewer rows than one workgroup, two rounds
    (n = 8192).  Edge data; the parity rule and, row by row, the bound; two
    launches bit for bit alike."""
    x, w = case(m, k, n, seed=7900 + n + k + m, edge=True)
    monkeypatch.setenv("DMC_HIP_RD_X8", "2")
    p = hip.plan("rd", m, k, n, x_addr=256, w_addr=256)
    assert (p.waves, p.rows_or_rw, p.rows_per_group, p.slices, p.mt, p.grid_x) == (4, 4, 16, 1, m, -(-n // 16)), p
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), _rd_dev(hip, x, w).view(np.uint32))
    check_or_bound(y, ref(x, w), x, W.bf16_to_f32(w), what=f"x4 m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("k", [2048, 1032])
def test_four_wave_group_zero_rule(hip, k, m, monkeypatch):
    """Exact zeros on the 4-wave group: the patterns of
    test_shared_x_fourteen_waves_zero_rule, bit for bit the reference."""
    monkeypatch.setenv("DMC_HIP_RD_X8", "2")
    n = 4096
    assert hip.plan("rd", m, k, n, x_addr=256, w_addr=256).waves == 4
    x = np.full((m, k), np.float32(-1e-38), np.float32)
    x[1::2] = -x[1::2]
    w = np.full((n, k), 0x0001, np.uint16)
    w[1::2, :] = 0x8001
    y_ref = ref(x, w)
    y = _rd_dev(hip, x, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
    xm, wz = zero_rows(k, 9)
    w = np.ascontiguousarray(wz[np.arange(n) % 9])
    xm = np.ascontiguousarray(xm[(2 + np.arange(m)) % 4])
    y_ref = ref(xm, w)
    y = _rd_dev(hip, xm, w)
    assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), \
        np.flatnonzero(y.view(np.uint32) != y_ref.view(np.uint32))[:8]


# ---- prefill-sized M on the gemm layout (16 * MB activation rows per workgroup) --------

@pytest.mark.parametrize("fuse", [0, 2])
@pytest.mark.parametrize("m,k,n", [(9, 512, 300), (16, 4096, 1000), (13, 64, 17),
                                   (17, 4096, 1000), (32, 64, 300), (33, 576, 257), (64, 4096, 513),
                                   (65, 1024, 700), (100, 14336, 260), (128, 4096, 4096), (200, 128, 17),
                                   (130, 1024, 600)])
def test_prefill_gemm_within_bound(hip, m, k, n, fuse, monkeypatch):
    """The gemm layout (the default from 17 rows on larger matrices, and at
    9..16 above 128 MiB): 16, 32 or 64 activation rows per workgroup, partial
    activation tiles (m = 9, 13, 17, 33, 65, 100, 130, 200), partial weight
    blocks, K from one chunk to 224, x split into planes by a launch
    (DMC_HIP_GEMM_FUSE=0) or by each workgroup (=2); edge data (subnormals,
    +-0, +-1e-38, inf/NaN weights).  Every element within the rigorous bound,
    non-finite classes and exact zeros as the reference."""
    x, w = case(m, k, n, seed=9000 + m + k + n, edge=True)
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "8")  # small matrices run rows16 by default
    monkeypatch.setenv("DMC_HIP_GEMM_FUSE", str(fuse))
    p = hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert (p.slices, p.mt) == (-8, 16 if m <= 16 else 32 if m <= 32 else 64), p
    y = run_rd(hip, x, w)
    rows = np.unique(np.r_[0, n - 1, np.random.default_rng(m).integers(0, n, 160)])
    y_ref = oracle.matmul_bf16_t(x, w[rows])
    check(y[:, rows], y_ref, what=f"gemm fuse={fuse} m={m} k={k} n={n}")
    wf = W.bf16_to_f32(w[rows])
    fin = np.all(np.isfinite(wf), axis=1)
    for r in range(0, m, 7):
        check_bound(y[r, rows[fin]], y_ref[r, fin], x[r], wf[fin], what=f"gemm fuse={fuse} m={m} k={k} n={n} row {r}")


@pytest.mark.parametrize("waves,m,k,n", [(4, 17, 4096, 1000), (4, 33, 576, 257), (4, 64, 4096, 513),
                                         (4, 100, 14336, 260), (4, 200, 128, 17), (4, 130, 1024, 600),
                                         (8, 17, 4096, 1000), (8, 24, 1024, 700), (8, 32, 64, 300)])
def test_prefill_gemm_four_and_eight_wave_workgroups(hip, waves, m, k, n, monkeypatch):
    """The gemm layout on 4-wave workgroups (128 weight rows, two per CU;
    DMC_HIP_GEMM_WAVES=4; the default at 32-row tiles on short grids), 32-
    and 64-row activation tiles: at 64 each thread stages two x items; and
    32-row tiles forced back onto 8-wave workgroups (C4's plan).  Partial
    weight and activation tiles, k split or not, edge data; every element
    within the rigorous bound, non-finite classes and exact zeros as the
    reference."""
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "8")
    monkeypatch.setenv("DMC_HIP_GEMM_WAVES", str(waves))
    x, w = case(m, k, n, seed=9300 + m + k + n, edge=True)
    w[min(3, n - 1)] = 0
    p = hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert (p.slices, p.mt, p.waves, p.rows_per_group) == (-8, 32 if m <= 32 else 64, waves, 32 * waves), p
    y = run_rd(hip, x, w)
    rows = np.unique(np.r_[0, min(3, n - 1), n - 1, np.random.default_rng(m).integers(0, n, 160)])
    y_ref = oracle.matmul_bf16_t(x, w[rows])
    check(y[:, rows], y_ref, what=f"gemm {waves} waves m={m} k={k} n={n}")
    wf = W.bf16_to_f32(w[rows])
    fin = np.all(np.isfinite(wf), axis=1)
    for r in range(0, m, 7):
        check_bound(y[r, rows[fin]], y_ref[r, fin], x[r], wf[fin], what=f"gemm {waves} waves m={m} k={k} n={n} row {r}")


@pytest.mark.parametrize("m,k,n", [(9, 1024, 700), (16, 4096, 513)])
def test_gemm_fused_single_slice_needs_no_workspace(hip, m, k, n, monkeypatch):
    """16-row activation tiles split x in the kernel, so with k in one slice
    (what the planner picks when the tiles alone fill the device, e.g. m =
    9..16 on 65k-98k rows) the plan has no workspace and the launch gets none:
    through the drop-in and through device pointers."""
    monkeypatch.setenv("DMC_HIP_GEMM_MAX_SLICES", "1")
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "8")
    x, w = case(m, k, n, seed=9700 + m + k + n, edge=True)
    p = hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert (p.slices, p.mt, p.workspace_bytes) == (-8, 16, 0), p
    y_ref = ref(x, w)
    check(run_rd(hip, x, w), y_ref, what=f"gemm fused unsplit m={m} k={k} n={n}")
    with hip.DeviceBuffer.from_numpy(w) as dw, hip.DeviceBuffer.from_numpy(x) as dx, \
            hip.DeviceBuffer(4 * m * n) as dy:
        hip.gemv_rd(dx, dw, dy, m, k, n)
        hip.synchronize()
        check(dy.download(np.float32, (m, n)), y_ref, what=f"gemm fused unsplit device m={m} k={k} n={n}")


@pytest.mark.parametrize("fuse", [0, 2])
@pytest.mark.parametrize("m,k,n", [(17, 4096, 1000), (64, 576, 513), (100, 1024, 260)])
def test_prefill_gemm_unsplit(hip, m, k, n, fuse, monkeypatch):
    """The gemm layout with k in one slice (DMC_HIP_GEMM_MAX_SLICES=1: what it
    runs when the tiles alone fill the device, as on the LM head), where the
    zero rule runs inside the kernel, with x split into planes by a launch
    (DMC_HIP_GEMM_FUSE=0) or by each workgroup (=2: no workspace at all):
    edge data, an all-zero weight row, and rows whose underflowing products
    end at -0.0 and +0.0."""
    monkeypatch.setenv("DMC_HIP_GEMM_MAX_SLICES", "1")
    monkeypatch.setenv("DMC_HIP_GEMM_FUSE", str(fuse))
    monkeypatch.setenv("DMC_HIP_RD_MFMA_KIND", "8")  # small matrices run rows16 by default
    x, w = case(m, k, n, seed=9500 + m + k + n, edge=True)
    w[3] = 0
    w[5] = 0x0001
    w[6] = 0x8001
    x[1] = np.float32(-1e-38)
    p = hip.plan("rd", m, k, n, x_addr=x.ctypes.data, w_addr=w.ctypes.data)
    assert p.slices == -8 and p.workspace_bytes == (0 if fuse else 3 * m * k * 2), p
    y = run_rd(hip, x, w)
    y_ref = ref(x, w)
    check(y, y_ref, what=f"gemm unsplit fuse={fuse} m={m} k={k} n={n}")
    assert np.signbit(y_ref[1, 5]) and np.signbit(y[1, 5]) and y[1, 5] == 0
    assert not np.signbit(y[1, 6]) and y[1, 6] == 0
