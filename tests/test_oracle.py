"""Pins for the CPU oracle (oracle/dmc_oracle.c), CPU only.

The oracle restates the reference's bf16 matmul (compiler/src/jit.rs:29481-29681).
Nothing here retypes its formula: each check compares it with something
independent --
  * the reference's own known-answer tests (widen, transpose, the m=3,k=5,n=4
    matmul, the ones sums) and exact-rational fma chains (tests/golden/);
  * a rigorous forward-error bound at the reference's large bit-exactness
    shape (jit.rs:30016-30030);
  * invariances the reference states: thread count (jit.rs:29501-29503),
    `x @ W'` == transpose-then-matmul, batched == per slice;
  * planted mistakes (oracle.mutation) that each of these must catch.
"""
import json
import math
import pathlib

import numpy as np
import pytest

import oracle
import exact_fma as E

GOLDEN = json.loads((pathlib.Path(__file__).parent / "golden" / "golden_vectors.json").read_text())


def u16(hexes):
    return np.array([int(h, 16) for h in hexes], np.uint16)


def f32(hexes):
    return np.array([int(h, 16) for h in hexes], np.uint32).view(np.float32)


def same_bits_nan_by_class(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def gemv_cases():
    return [c["name"] for c in GOLDEN["gemv"]]


def load_case(name):
    c = next(c for c in GOLDEN["gemv"] if c["name"] == name)
    x = np.array([f32(r) for r in c["x"]], np.float32).reshape(c["m"], c["k"])
    w = np.array([u16(r) for r in c["w_nk"]], np.uint16).reshape(c["n"], c["k"])
    out = np.array([f32(r) for r in c["out"]], np.float32).reshape(c["m"], c["n"])
    return x, w, out


# ---- golden vectors ---------------------------------------------------------------

def test_widen_kat():
    g = GOLDEN["widen"]
    assert np.array_equal(oracle.widen(u16(g["in"])).view(np.uint32),
                          np.array([int(h, 16) for h in g["out"]], np.uint32))


def test_truncate_kat():
    g = GOLDEN["truncate"]
    assert np.array_equal(oracle.truncate(f32(g["in"])), u16(g["out"]))


def test_transpose_kat():
    g = GOLDEN["transpose"]
    src = u16(g["in"]).reshape(g["m"], g["n"])
    assert np.array_equal(oracle.transpose(src).reshape(-1), u16(g["out"]))


@pytest.mark.parametrize("name", gemv_cases())
def test_gemv_golden_both_layouts(name):
    x, w, out = load_case(name)
    y_cs = oracle.matmul_bf16(x, np.ascontiguousarray(w.T))
    y_rd = oracle.matmul_bf16_t(x, w)
    assert same_bits_nan_by_class(y_cs, out), (name, y_cs, out)
    assert same_bits_nan_by_class(y_rd, out), (name, y_rd, out)
    mi, ni = np.meshgrid(np.arange(x.shape[0]), np.arange(w.shape[0]), indexing="ij")
    for lay, wl in (("rd", w), ("cs", np.ascontiguousarray(w.T))):
        pts = oracle.gemv_points(x, wl, lay, mi.reshape(-1), ni.reshape(-1))
        assert same_bits_nan_by_class(pts, out.reshape(-1)), (name, lay)


def test_reference_kat_sums():
    # jit.rs:42643-42655 asserts sum(x @ w) == 6; jit_probes.py:932 asserts 4
    x, w, _ = load_case("jit_bf16_field_matmul_ones")
    assert oracle.matmul_bf16_t(x, w).sum() == 6
    x, w, _ = load_case("probe_matmul_1xN_Nx1")
    assert oracle.matmul_bf16_t(x, w)[0, 0] == 4


def test_exact_fma_agrees_with_hardware_on_random_triples():
    # the checker itself against the host's correctly rounded fmaf (via the
    # oracle's k = 1 chain: fma(x, w, +0)) and against numpy's exact products
    rng = np.random.default_rng(1)
    x = rng.standard_normal(2000).astype(np.float32) * np.float32(1e3)
    w = ((rng.standard_normal(2000).astype(np.float32).view(np.uint32) + 0x7FFF) >> 16).astype(np.uint16)
    got = oracle.gemv_points(x.reshape(-1, 1), w.reshape(-1, 1), "rd",
                             np.arange(2000), np.arange(2000))
    want = np.array([E.fma(float(a), E.bf16_to_f32(int(h)), 0.0) for a, h in zip(x, w)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- size-independent properties ---------------------------------------------------

def large_pin_inputs():
    """jit.rs:30016-30030: k=2560, n=9728, a[i] = (i%13) as f32 * 0.1,
    b[i] = 0x3f00 | (i & 0x7f)."""
    k, n = 2560, 9728
    a = (np.arange(k) % 13).astype(np.float32) * np.float32(0.1)
    b = (0x3F00 | (np.arange(k * n) & 0x7F)).astype(np.uint16).reshape(k, n)
    return a, b, k, n


def test_large_shape_forward_error_bound():
    """|y - exact| <= gamma_k * sum|a*w| for every column of the reference's
    large bit-exactness shape, with the exact value from float64 fsum (the
    products are exact in binary64: 24 x 8 significant bits)."""
    a, b, k, n = large_pin_inputs()
    y = oracle.matmul_bf16(a, b)[0].astype(np.float64)
    wf = oracle.widen(b).astype(np.float64)
    prods = a.astype(np.float64)[:, None] * wf
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    cols = np.arange(0, n, 37)
    for j in cols:
        exact = math.fsum(prods[:, j])
        bound = gamma * np.abs(prods[:, j]).sum()
        assert abs(y[j] - exact) <= bound, (j, y[j], exact, bound)
    # and it is the ascending chain: a dropped/reordered term moves it off the
    # exact sum by more than rounding (checked under mutation below)


@pytest.mark.parametrize("workers", [1, 2, 3, 4, 7])
def test_thread_count_invariance(workers):
    a, b, k, n = large_pin_inputs()
    base = oracle.matmul_bf16(a, b, workers=1)
    assert np.array_equal(oracle.matmul_bf16(a, b, workers=workers).view(np.uint32),
                          base.view(np.uint32))
    x = np.random.default_rng(2).standard_normal((5, 300)).astype(np.float32)
    w = b[:300, :700].copy()
    ref = oracle.matmul_bf16(x, w, workers=1)
    assert np.array_equal(oracle.matmul_bf16(x, w, workers=workers).view(np.uint32), ref.view(np.uint32))


def test_rowdot_equals_transpose_then_matmul():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 517)).astype(np.float32)
    w = ((rng.standard_normal((129, 517)).astype(np.float32).view(np.uint32)) >> 16).astype(np.uint16)
    assert np.array_equal(oracle.matmul_bf16_t(x, w).view(np.uint32),
                          oracle.matmul_bf16(x, oracle.transpose(w)).view(np.uint32))


def test_batched_equals_per_slice():
    rng = np.random.default_rng(4)
    k, n, batch, ls, rs = 40, 24, 5, 48, 40 * 24 + 8
    x = rng.standard_normal((batch - 1) * ls + k).astype(np.float32)
    w = (rng.integers(0, 1 << 16, (batch - 1) * rs + k * n)).astype(np.uint16) & 0xBFFF
    out = oracle.matmul_bf16_batched(x, w, k, n, batch, ls, rs)
    for z in range(batch):
        ref = oracle.matmul_bf16(x[z * ls:z * ls + k], w[z * rs:z * rs + k * n].reshape(k, n))[0]
        assert same_bits_nan_by_class(out[z * n:(z + 1) * n], ref)


def test_k_zero_writes_positive_zero_and_m_n_zero_noop():
    y = oracle.matmul_bf16(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.uint16))
    assert np.all(y == 0) and not np.signbit(y).any()


# ---- threading policy (jit.rs:29467-29479, 29527-29529) ------------------------------

def test_gemv_ways_policy(monkeypatch):
    monkeypatch.delenv("DMC_BF16_COLSPLIT", raising=False)
    # thresholds in weight bytes, both sides of each boundary
    assert oracle.gemv_ways(1024, 1023) == 1                # 2 MiB - 2 KiB
    assert oracle.gemv_ways(1024, 1024) == 2                # exactly 2 MiB
    assert oracle.gemv_ways(4096, 2048) == 4                # exactly 16 MiB
    assert oracle.gemv_ways(4096, 2047) == 2
    monkeypatch.setenv("DMC_BF16_COLSPLIT", "0")
    assert oracle.gemv_ways(4096, 14336) == 1


def test_matmul_threads_policy(monkeypatch):
    monkeypatch.setenv("DMC_MATMUL_THREADS", "6")
    assert oracle.matmul_threads(1, 4096, 4096) == 1        # m < 2
    assert oracle.matmul_threads(2, 512, 1023) == 1         # < 2^20 MACs
    assert oracle.matmul_threads(2, 512, 1024) == 2         # capped by m
    assert oracle.matmul_threads(64, 512, 512) == 6


# ---- the pins have teeth: every planted mistake is caught --------------------------------

def pins_pass() -> bool:
    ok = True
    for name in gemv_cases():
        x, w, out = load_case(name)
        ok &= same_bits_nan_by_class(oracle.matmul_bf16(x, np.ascontiguousarray(w.T)), out)
    g = GOLDEN["widen"]
    ok &= np.array_equal(oracle.widen(u16(g["in"])).view(np.uint32),
                         np.array([int(h, 16) for h in g["out"]], np.uint32))
    return bool(ok)


@pytest.mark.parametrize("mut", sorted(oracle.MUTATIONS))
def test_planted_mistake_is_caught(mut):
    assert pins_pass()
    with oracle.mutation(mut):
        assert not pins_pass(), f"mutation {mut} slipped through the golden pins"
    assert pins_pass()
