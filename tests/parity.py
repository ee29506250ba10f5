"""The parity rule shared by every GPU test.

Reference values come from the oracle (the reference's ascending-k fmaf
chain).  Device results must match
  * the non-finite class exactly (NaN <-> NaN, +inf <-> +inf, -inf <-> -inf;
    NaN payload and sign are not compared),
  * exact zeros bitwise (value and sign) wherever the reference is 0,
  * normwise over the finite reference outputs:
        ||y - y_ref||_2 / ||y_ref||_2 <= 1e-5
    (the tolerance the north star states for a different accumulation order;
    the expected gap at K = 14336 is ~3e-6).
"""
import numpy as np

TOL = 1e-5


def check(y, y_ref, tol=TOL, what=""):
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
    d = (y[fin].astype(np.float64) - y_ref[fin].astype(np.float64))
    nr = np.linalg.norm(y_ref[fin].astype(np.float64))
    nd = np.linalg.norm(d)
    if nr == 0:
        assert nd == 0, f"{what}: reference is all zero, device differs by {nd}"
        return 0.0
    rel = nd / nr
    assert rel <= tol, f"{what}: normwise relative error {rel:.3e} > {tol:.0e}"
    return rel
