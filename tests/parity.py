"""The parity rule shared by every GPU test.

Reference values come from the oracle (the reference's ascending-k fmaf
chain).  Device results must match
  * the non-finite class exactly (NaN <-> NaN, +inf <-> +inf, -inf <-> -inf;
    NaN payload and sign are not compared), and be finite wherever the
    reference is finite,
  * exact zeros bitwise (value and sign) wherever the reference is 0,
  * normwise over the finite reference outputs:
        ||y - y_ref||_2 / ||y_ref||_2 <= 1e-5
    (the tolerance the north star states for a different accumulation order;
    the expected gap at K = 14336 is ~3e-6).
Rows that edge data leaves ill-conditioned (cancellation, or products with
inf/NaN weights elsewhere in the batch) are held instead to the rigorous
elementwise forward-error bound of two fma chains over the same products in
different orders (`check_bound`), with the same class and zero rules.

Every comparison is written so that a NaN fails it: `not (err <= bound)`,
never `err > bound`.  tests/test_parity_rule.py plants a NaN, an inf of
either sign, a flipped zero and an out-of-bound value and requires each
checker here to reject it.
"""
import numpy as np

TOL = 1e-5


def check_classes(y, y_ref, what=""):
    """Non-finite classes, finiteness and exact zeros (the part of the rule
    that no tolerance relaxes)."""
    y = np.asarray(y, np.float32)
    y_ref = np.asarray(y_ref, np.float32)
    assert y.shape == y_ref.shape, (what, y.shape, y_ref.shape)
    nan_r, nan_y = np.isnan(y_ref), np.isnan(y)
    assert np.array_equal(nan_r, nan_y), \
        f"{what}: NaN class mismatch at {np.flatnonzero(nan_r != nan_y)[:8]}"
    for sgn in (1, -1):
        ir = np.isinf(y_ref) & (np.sign(y_ref) == sgn)
        iy = np.isinf(y) & (np.sign(y) == sgn)
        assert np.array_equal(ir, iy), \
            f"{what}: {'+' if sgn > 0 else '-'}inf mismatch at {np.flatnonzero(ir != iy)[:8]}"
    fin = np.isfinite(y_ref)
    assert np.all(np.isfinite(y[fin])), f"{what}: non-finite output where reference is finite"
    z = fin & (y_ref == 0)
    if z.any():
        bad = z & ((y != 0) | (np.signbit(y) != np.signbit(y_ref)))
        assert not bad.any(), f"{what}: signed-zero mismatch at {np.flatnonzero(bad)[:8]}: " \
            f"{y[bad][:4]} vs {y_ref[bad][:4]}"
    return fin


def check(y, y_ref, tol=TOL, what=""):
    y = np.asarray(y, np.float32)
    y_ref = np.asarray(y_ref, np.float32)
    fin = check_classes(y, y_ref, what)
    d = (y[fin].astype(np.float64) - y_ref[fin].astype(np.float64))
    nr = np.linalg.norm(y_ref[fin].astype(np.float64))
    nd = np.linalg.norm(d)
    if nr == 0:
        assert nd == 0, f"{what}: reference is all zero, device differs by {nd}"
        return 0.0
    rel = nd / nr
    assert rel <= tol, f"{what}: normwise relative error {rel:.3e} > {tol:.0e}"
    return rel


def check_bound(y, y_ref, x, w_rows, what=""):
    """Elementwise: |y - y_ref| <= 2*K*u*sum_k |x_k * w_k| (u = 2^-24) for every
    finite reference output -- the rigorous forward-error bound of two
    length-K fma chains of the same products in different orders -- plus the
    class and zero rules.  x is the activation row, w_rows the widened
    weights of the checked outputs [n, K]."""
    fin = check_classes(y, y_ref, what)
    y = np.asarray(y, np.float64)
    y_ref = np.asarray(y_ref, np.float64)
    k = x.shape[-1]
    s = np.abs(w_rows.astype(np.float64)) @ np.abs(x.astype(np.float64))
    bound = 2 * k * 2.0 ** -24 * s + 2.0 ** -149
    with np.errstate(invalid="ignore"):
        bad = fin & ~(np.abs(y - y_ref) <= bound)
    assert not bad.any(), f"{what}: error beyond the rigorous bound at {np.flatnonzero(bad)[:8]}"


def check_or_bound(y, y_ref, x, wf, what=""):
    """The parity rule for a batch [m, n]; when the normwise rule fails
    (edge data: ill-conditioned rows, inf/NaN weights), every output is held
    to the class and zero rules and each row whose weights are finite to
    the elementwise bound.  x [m, K] activations, wf [n, K] widened weights."""
    try:
        check(y, y_ref, what=what)
    except AssertionError:
        check_classes(y, y_ref, what)
        fin = np.all(np.isfinite(wf), axis=1)
        for r in range(y.shape[0]):
            check_bound(y[r, fin], y_ref[r, fin], x[r], wf[fin], what=f"{what} row {r}")
