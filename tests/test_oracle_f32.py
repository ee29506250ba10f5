"""Pins for the f32 oracle (oracle_matmul_f32, oracle_gemv_points_f32), CPU only.

The oracle restates the reference's f32 `@` (dmc_matmul_par's matmul_tile,
compiler/src/jit.rs:29448-29466, bit-identical to scalar_matmul / simd_matmul,
jit.rs:20525-20802).  Each check compares it with something independent:
  * the reference's own f32 matmul tests, restated as data: the contraction
    test (jit.rs:37386-37420: the fused answer differs from a two-rounding hand
    loop), the unrelated-columns test (jit.rs:37353-37384: C[0,0] does not move
    with B's width), and the scalar/SIMD path sums (jit.rs:34311-34337);
  * an exact-rational fma chain (tests/exact_fma.py) on small cases with
    subnormals, signed zeros, inf and NaN;
  * the already-pinned bf16 oracle on bf16-representable weights (the same
    closed form through another code path);
  * planted mistakes (oracle.mutation) that these pins must catch.
"""
import math

import numpy as np
import pytest

import oracle
import exact_fma as E


def f32_expr_a(i, j):
    """((i*16+j) as f32 * 0.7f32 + 0.1f32) / 3.0f32, each operation rounded to f32."""
    v = np.float32(i * 16 + j) * np.float32(0.7)
    return (v + np.float32(0.1)) / np.float32(3.0)


def f32_expr_b(i, j, stride):
    """((i*stride+j) as f32 * 0.3f32 + 0.2f32) / 7.0f32, each operation rounded to f32."""
    v = np.float32(i * stride + j) * np.float32(0.3)
    return (v + np.float32(0.2)) / np.float32(7.0)


def contraction_case(n=16, stride=16):
    a = np.array([[f32_expr_a(i, j) for j in range(16)] for i in range(8)], np.float32)
    b = np.array([[f32_expr_b(i, j, stride) for j in range(n)] for i in range(16)], np.float32)
    return a, b


def bits(v):
    return np.asarray(v, np.float32).view(np.uint32)


def exact(l, r):
    """The reference chain per element, exactly (small cases only)."""
    m, k = l.shape
    n = r.shape[1]
    out = np.empty((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            out[i, j] = E.chain([float(v) for v in l[i]], [float(v) for v in r[:, j]])
    return out


def same_nan_by_class(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(bits(a)[~na], bits(b)[~nb]))


def edge_case(seed, m, k, n):
    rng = np.random.default_rng(seed)
    l = rng.standard_normal((m, k)).astype(np.float32)
    r = rng.standard_normal((k, n)).astype(np.float32)
    specials = np.array([0.0, -0.0, 1e-38, -1e-38, 1e-45, -1e-45, np.inf, -np.inf, np.nan, 3e38], np.float32)
    for a in (l, r):
        flat = a.reshape(-1)
        pos = rng.integers(0, flat.size, size=max(1, flat.size // 6))
        flat[pos] = rng.choice(specials, size=pos.size)
    return l, r


def pin_set():
    """Small cases the pins compare against the exact chain: random data with
    special values, an all-zero activation row, underflowing products of both
    signs (zero signs), a non-square weight."""
    cases = [edge_case(s, 3, 7, 5) for s in range(4)]
    l = np.zeros((2, 6), np.float32)
    l[1] = np.float32(1e-30)
    r = np.full((6, 3), np.float32(1e-30), np.float32)
    r[:, 1] = -r[:, 1]
    r[::2, 2] = -r[::2, 2]
    cases.append((l, r))
    return cases


def pins_pass() -> bool:
    ok = True
    for l, r in pin_set():
        ok &= same_nan_by_class(oracle.matmul_f32(l, r), exact(l, r))
    a, b = contraction_case()
    two = np.float32(0.0)
    for i in range(16):
        two = np.float32(two + np.float32(a[0, i] * b[i, 0]))
    c00 = oracle.matmul_f32(a, b)[0, 0]
    ok &= bits(c00) != bits(two)
    ok &= bool(bits(oracle.matmul_f32(np.ones((1, 0), np.float32)[:, :0], np.ones((0, 2), np.float32)))[0, 0] == 0)
    return bool(ok)


# ---- the reference's own f32 matmul tests ---------------------------------------------

def test_contraction_kat():
    """jit.rs:37386-37420: the fused chain and a two-rounding loop differ on this
    data; the oracle is the fused one, equal to the exact chain."""
    a, b = contraction_case()
    c = oracle.matmul_f32(a, b)
    want = E.chain([float(v) for v in a[0]], [float(v) for v in b[:, 0]])
    assert bits(c[0, 0]) == bits(np.float32(want))
    two = np.float32(0.0)
    for i in range(16):
        two = np.float32(two + np.float32(a[0, i] * b[i, 0]))
    assert bits(c[0, 0]) != bits(two)


def test_result_does_not_depend_on_unrelated_columns():
    """jit.rs:37353-37384: C[0,0] for B [16, n] with b[i,j] from i*97+j is the
    same for n = 3, 4, 15, 16."""
    got = {n: oracle.matmul_f32(*contraction_case(n, 97))[0, 0] for n in (3, 4, 15, 16)}
    assert len({int(bits(v)) for v in got.values()}) == 1, got


def test_scalar_and_simd_path_sums():
    """jit.rs:34311-34337: sum(a @ b) on small integer matrices, against
    integer arithmetic."""
    a = np.array([[1, 2, 3], [4, 5, 6]])
    b = np.array([[7, 8, 9], [1, 2, 3], [4, 5, 6]])
    assert oracle.matmul_f32(a.astype(np.float32), b.astype(np.float32)).sum() == (a @ b).sum()
    a = np.array([[2, 3, 5, 7], [11, 13, 17, 19]])
    b = np.arange(1, 17).reshape(4, 4)
    assert oracle.matmul_f32(a.astype(np.float32), b.astype(np.float32)).sum() == (a @ b).sum()


# ---- independent restatements ---------------------------------------------------------

@pytest.mark.parametrize("case", range(5))
def test_exact_chain_with_special_values(case):
    l, r = pin_set()[case]
    assert same_nan_by_class(oracle.matmul_f32(l, r), exact(l, r))


def test_zero_signs_follow_the_chain():
    # every product underflows: negative ones end at -0, positive at +0,
    # alternating signs at the sign of the last; an all-zero row stays +0
    l, r = pin_set()[4]
    y = oracle.matmul_f32(l, r)
    assert np.all(y[0] == 0) and not np.any(np.signbit(y[0]))
    assert y[1, 0] == 0 and not np.signbit(y[1, 0])
    assert y[1, 1] == 0 and np.signbit(y[1, 1])
    assert y[1, 2] == 0 and np.signbit(y[1, 2]) == (r[-1, 2] < 0)


@pytest.mark.parametrize("seed", [0, 1])
def test_equals_bf16_oracle_on_bf16_weights(seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((3, 300)).astype(np.float32)
    w = ((rng.standard_normal((300, 40)).astype(np.float32).view(np.uint32) + 0x7FFF) >> 16).astype(np.uint16)
    w.reshape(-1)[rng.integers(0, w.size, 20)] = 0x0001  # subnormal bf16 weights
    a = oracle.matmul_f32(x, oracle.widen(w))
    b = oracle.matmul_bf16(x, w)
    assert np.array_equal(bits(a), bits(b))


def test_points_equal_full_product():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 97)).astype(np.float32)
    w_nk = rng.standard_normal((33, 97)).astype(np.float32)
    full = oracle.matmul_f32(x, np.ascontiguousarray(w_nk.T))
    mi = rng.integers(0, 4, 50)
    ni = rng.integers(0, 33, 50)
    assert np.array_equal(bits(oracle.gemv_points_f32(x, w_nk, mi, ni)), bits(full[mi, ni]))


def test_k_zero_writes_positive_zero_and_empty_is_noop():
    y = oracle.matmul_f32(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.float32))
    assert y.shape == (2, 3) and np.all(y == 0) and not np.any(np.signbit(y))
    assert oracle.matmul_f32(np.zeros((0, 4), np.float32), np.zeros((4, 3), np.float32)).shape == (0, 3)


def test_large_shape_forward_error_bound():
    """|y - exact| <= gamma_k * sum|l*r| at a decode-like size, the exact value
    from float64 fsum of the exactly representable products (24 x 24 bits)."""
    rng = np.random.default_rng(4)
    k = 4096
    x = rng.standard_normal(k).astype(np.float32)
    w = rng.standard_normal((k, 64)).astype(np.float32)
    y = oracle.matmul_f32(x, w)[0].astype(np.float64)
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    for j in range(64):
        prods = x.astype(np.float64) * w[:, j].astype(np.float64)
        ex = math.fsum(prods)
        assert abs(y[j] - ex) <= gamma * np.abs(prods).sum()


# ---- the pins have teeth ------------------------------------------------------------------

@pytest.mark.parametrize("mut", ["drop_last_k", "neg_zero_init", "unfused", "transposed_w", "descending_k"])
def test_planted_mistake_is_caught(mut):
    assert pins_pass()
    with oracle.mutation(mut):
        assert not pins_pass(), f"mutation {mut} slipped through the f32 pins"
    assert pins_pass()
