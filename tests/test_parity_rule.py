"""The parity checkers themselves, on the CPU: each planted mistake must fail.

A checker that accepts a wrong output pins nothing, so every rule of
tests/parity.py is exercised both ways here -- a correct device-like result
passes, and a NaN where the reference is finite, an inf of either sign, a
flipped zero sign, a wrong non-finite class and an out-of-bound value each
raise -- for `check`, `check_bound` and `check_or_bound` (the random sweep's
rule, including its fallback for ill-conditioned rows).
"""
import numpy as np
import pytest

import oracle
from demonic_amd import workloads as W
from parity import check, check_bound, check_classes, check_or_bound


def _case(ill=False):
    rng = np.random.default_rng(5)
    m, k, n = 3, 256, 40
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = W.bf16_rne(rng.standard_normal((n, k)).astype(np.float32) * 0.02).reshape(n, k)
    if ill:
        # Row 0 cancels: its true values are tiny against sum |x w|, so a
        # result within the rigorous bound misses the normwise rule.
        x[0, : k // 2] = 1e4
        x[0, k // 2:] = -1e4
        w[:, k // 2:] = w[:, : k // 2]
    y_ref = oracle.matmul_bf16_t(x, w)
    return x, w, W.bf16_to_f32(w), y_ref


def _plants(y_ref):
    """(name, planted output) pairs, each of which breaks the rule."""
    out = []
    last = y_ref[-1]  # a well-conditioned row in both cases
    i = y_ref.size - last.size + int(np.flatnonzero(np.isfinite(last) & (last != 0))[0])
    for name, v in (("nan", np.nan), ("+inf", np.inf), ("-inf", -np.inf)):
        y = y_ref.copy()
        y.ravel()[i] = v
        out.append((name, y))
    y = y_ref.copy()
    y.ravel()[i] = y_ref.ravel()[i] * (1 + 1e-2) + 1e-3  # far outside both rules
    out.append(("off", y))
    return out


def test_correct_result_passes():
    x, w, wf, y_ref = _case()
    y = y_ref.copy()
    y[np.abs(y) > 0] = np.nextafter(y[np.abs(y) > 0], np.float32(np.inf))  # one ulp: inside every rule
    check(y, y_ref)
    for r in range(y.shape[0]):
        check_bound(y[r], y_ref[r], x[r], wf)
    check_or_bound(y, y_ref, x, wf)


@pytest.mark.parametrize("ill", [False, True])
def test_planted_mistakes_fail_every_checker(ill):
    x, w, wf, y_ref = _case(ill)
    for name, y in _plants(y_ref):
        with pytest.raises(AssertionError):
            check(y, y_ref, what=name)
        with pytest.raises(AssertionError):
            for r in range(y.shape[0]):
                check_bound(y[r], y_ref[r], x[r], wf, what=name)
        with pytest.raises(AssertionError):
            check_or_bound(y, y_ref, x, wf, what=name)


def test_ill_conditioned_row_takes_the_fallback():
    """Row 0 of the ill case misses the normwise rule by design; a result
    within the elementwise bound passes check_or_bound, so the fallback is
    really exercised by the planted cases above."""
    x, w, wf, y_ref = _case(ill=True)
    s = np.abs(wf.astype(np.float64)) @ np.abs(x[0].astype(np.float64))
    y = y_ref.copy()
    nz = y_ref[0] != 0  # exact zeros keep their bits (the zero rule)
    y[0, nz] = (y_ref[0, nz] + 0.25 * 2 * x.shape[1] * 2.0 ** -24 * s[nz]).astype(np.float32)
    with pytest.raises(AssertionError):
        check(y, y_ref)
    check_or_bound(y, y_ref, x, wf)


def test_zero_sign_and_nan_class():
    y_ref = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1.0], np.float32)
    check_classes(y_ref.copy(), y_ref)
    for i, v in ((0, -0.0), (1, 0.0), (2, 1.0), (3, -np.inf), (4, np.nan), (5, np.nan), (5, np.inf), (0, 1e-45)):
        y = y_ref.copy()
        y[i] = v
        with pytest.raises(AssertionError):
            check_classes(y, y_ref)
    x = np.ones((1, 6), np.float32)
    wf = np.ones((6, 6), np.float32)
    y = y_ref.copy()
    y[0] = -0.0
    with pytest.raises(AssertionError):
        check_bound(y, y_ref, x[0], wf)
