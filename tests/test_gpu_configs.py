"""GPU parity at the full size of two BASELINE configurations.

C4: the LM head W [128256, 4096] (1.05 GB) at M = 1, 2, 4, 8, 12, 16, each M
on the kernel its real shape plans (streaming at M = 1 and 2, rows16 with two
blocks per workgroup at 4 and 8, the gemm MFMA layout with x split in the
kernel and k in one slice at 12 and 16).  C3: the whole
32-layer Llama-3-8B decode sweep (13.97 GB of weights), scheduled as the bench
runs it, every projection of every layer sampled with that layer's own x.

Weights are generated in HBM by the counter generator (dmc_hip_fill_counter_bf16);
the sampled rows are regenerated on the host bit for bit
(tests/test_gpu_parity.py::test_device_fill_matches_host_generator) and
checked against the oracle (the reference chain, jit.rs:29481-29681).
"""
import numpy as np
import pytest

import oracle
from demonic_amd import workloads as W
from parity import check, check_bound

pytestmark = pytest.mark.gpu

# M -> (kind, rows per workgroup) the real C4 shape must plan: kind is the
# streaming kernel's windows per lane (> 0) or -(MFMA layout) (7 rows16, 8 gemm)
# (slices, rows per workgroup): the streaming kernel at m = 1, the 8-wave group
# (16 rows, x in registers) at 2 to 4, the gemm layout from 6
C4_PLANS = {1: (1, 4), 2: (1, 16), 3: (1, 16), 4: (1, 16), 6: (-8, 256), 8: (-8, 256), 12: (-8, 256),
            16: (-8, 256)}


@pytest.fixture(scope="module")
def c4_weight(hip):
    n, k = W.LM_HEAD
    table = hip.DeviceBuffer.from_numpy(W.normal_table(0.02))
    dw = hip.DeviceBuffer(2 * n * k)
    hip.fill_counter_bf16(dw, n * k, W.counter_seed(0, W.C4_TENSOR), table)
    hip.synchronize()
    yield dw
    dw.free()
    table.free()


@pytest.mark.parametrize("m", sorted(C4_PLANS))
def test_c4_full_lm_head(hip, c4_weight, m):
    n, k = W.LM_HEAD
    x = np.random.default_rng(400 + m).standard_normal((m, k)).astype(np.float32)
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer(4 * m * n) as dy:
        p = hip.plan("rd", m, k, n, x_addr=dx.addr, w_addr=c4_weight.addr)
        assert (p.slices, p.rows_per_group) == C4_PLANS[m], p
        dy.upload(np.full(m * n, np.nan, np.float32))
        hip.gemv_rd(dx, c4_weight, dy, m, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (m, n))
    # 512 random rows, the first and last, and the last row of every
    # 256-row block (the gemm layout's workgroup boundary)
    rng = np.random.default_rng(m)
    rows = np.unique(np.r_[0, n - 1, rng.integers(0, n, 512), np.arange(255, n, 256)])
    wr = W.counter_rows(0, W.C4_TENSOR, rows, k, 0.02)
    y_ref = oracle.matmul_bf16_t(x, wr)
    rel = check(y[:, rows], y_ref, what=f"C4 m={m}")
    wf = W.bf16_to_f32(wr)
    for r in range(m):
        check_bound(y[r, rows], y_ref[r], x[r], wf, what=f"C4 m={m} row {r}")
    assert np.all(np.isfinite(y))
    print(f"C4 m={m} plan={p} rows={rows.size} rel={rel:.3e}")


@pytest.mark.parametrize("m", [4, 8, 16])
def test_c4_tiny_activation_rows(hip, c4_weight, m):
    """C4 at the plans its real shape takes (the 8-wave group at M = 4, the
    gemm layout at 8 and 16) with activation rows of N(0,1) * 1e-36 and *
    1e-37 beside ordinary rows (tests/test_gpu_tiny_rows.py: the rows the
    MFMA kernels' three-term split alone cannot carry): every row within the
    1e-5 normwise rule on its own, and on the MFMA plans the tiny rows bit for
    bit the reference chain (k is not split on these plans)."""
    from test_gpu_tiny_rows import check_rows, tiny_rows_x
    n, k = W.LM_HEAD
    x = tiny_rows_x(m, k, seed=500 + m)
    with hip.DeviceBuffer.from_numpy(x) as dx, hip.DeviceBuffer(4 * m * n) as dy:
        p = hip.plan("rd", m, k, n, x_addr=dx.addr, w_addr=c4_weight.addr)
        assert (p.slices, p.rows_per_group) == C4_PLANS[m] and p.workspace_bytes == 0, p
        dy.upload(np.full(m * n, np.nan, np.float32))
        hip.gemv_rd(dx, c4_weight, dy, m, k, n)
        hip.synchronize()
        y = dy.download(np.float32, (m, n))
    rows = np.unique(np.r_[0, n - 1, np.random.default_rng(m).integers(0, n, 256), np.arange(255, n, 4096)])
    wr = W.counter_rows(0, W.C4_TENSOR, rows, k, 0.02)
    check_rows(y[:, rows], oracle.matmul_bf16_t(x, wr), m, f"C4 tiny rows m={m}", exact=C4_PLANS[m][0] < 0)
    assert np.all(y[-1] == 0) and not np.any(np.signbit(y[-1]))


def test_c3_every_layer(hip):
    """One decode token of C3 as bench.py runs it (all 32 layers resident;
    q/k/v and gate/up grouped, o and down single; captured in a HIP graph and
    replayed), then every projection of every layer checked on ~40 sampled
    rows plus its first and last, against that layer's own activations."""
    names = [nm for nm, _, _ in W.LLAMA3_8B_LAYER]
    shape = {nm: (n, k) for nm, n, k in W.LLAMA3_8B_LAYER}
    table = hip.DeviceBuffer.from_numpy(W.normal_table(W.C3_SCALE))
    layers = []
    try:
        for layer in range(W.LLAMA3_8B_LAYERS):
            ws = {}
            for idx, nm in enumerate(names):
                n, k = shape[nm]
                ws[nm] = hip.DeviceBuffer(2 * n * k)
                hip.fill_counter_bf16(ws[nm], n * k, W.counter_seed(0, W.c3_tensor(layer, idx)), table)
            ys = {nm: hip.DeviceBuffer(4 * shape[nm][0]) for nm in names}
            layers.append((ws, ys, hip.DeviceBuffer.from_numpy(W.c3_x(layer, 4096)),
                           hip.DeviceBuffer.from_numpy(W.c3_x(layer, 14336))))

        def token():
            for ws, ys, dx, dx2 in layers:
                hip.gemv_rd_grouped([dx] * 3, [ws["q"], ws["k"], ws["v"]], [ys["q"], ys["k"], ys["v"]],
                                    [4096, 1024, 1024], 1, 4096)
                hip.gemv_rd(dx, ws["o"], ys["o"], 1, 4096, 4096)
                hip.gemv_rd_grouped([dx] * 2, [ws["gate"], ws["up"]], [ys["gate"], ys["up"]], [14336] * 2, 1, 4096)
                hip.gemv_rd(dx2, ws["down"], ys["down"], 1, 14336, 4096)

        token()
        hip.synchronize()
        g = hip.Graph()
        with g:
            token()
        try:
            for _, ys, _, _ in layers:
                for b in ys.values():
                    b.upload(np.full(b.nbytes // 4, np.nan, np.float32))
            g.launch()
            hip.synchronize()
        finally:
            g.destroy()
        worst = 0.0
        for layer, (_, ys, _, _) in enumerate(layers):
            rng = np.random.default_rng(1000 + layer)
            x, x2 = W.c3_x(layer, 4096), W.c3_x(layer, 14336)
            for idx, nm in enumerate(names):
                n, k = shape[nm]
                rows = np.unique(np.r_[0, n - 1, rng.integers(0, n, 40)])
                y = ys[nm].download(np.float32, (n,))
                assert np.all(np.isfinite(y)), (layer, nm)
                y_ref = oracle.matmul_bf16_t(x2 if nm == "down" else x, W.c3_rows(layer, idx, rows))[0]
                worst = max(worst, check(y[rows], y_ref, what=f"C3 layer {layer} {nm}"))
        print(f"C3 all 32 layers: worst rel={worst:.3e}")
    finally:
        for ws, ys, dx, dx2 in layers:
            for b in list(ws.values()) + list(ys.values()) + [dx, dx2]:
                b.free()
        table.free()
