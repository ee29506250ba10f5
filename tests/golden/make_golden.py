"""Write tests/golden/golden_vectors.json: inputs and exact expected outputs.

Sources of truth, none of them the oracle under test:
  * the reference's own known-answer tests, with the inputs they fully
    specify (compiler/src/jit.rs:30171-30178 widen, jit.rs:30204-30243 the
    m=3,k=5,n=4 bf16 matmul, jit.rs:30249-30263 transpose, jit.rs:42643-42655
    and tools/jit_probes.py:932 the ones sums);
  * exact-rational fused multiply-add chains (tests/exact_fma.py) for the
    expected GEMV outputs, including NaN/inf/signed-zero/subnormal edge cases.

Run from the repo root:  python tests/golden/make_golden.py
All values are stored as hex bit patterns.
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import exact_fma as E  # noqa: E402


def hx(vals, width):
    return [format(int(v), f"0{width}x") for v in vals]


def f32hex(xs):
    return hx([E.f32_bits(float(x)) for x in xs], 8)


def trunc_bf16(f: float) -> int:
    """jit.rs:30215-30216: (f.to_bits() >> 16) of an f32."""
    return E.f32_bits(f) >> 16


def f32(x: float) -> float:
    return float(np.float32(x))


def gemv_case(name, x_rows, w_logical, note):
    """x [m][k] f32 values, w_logical [n][k] bf16 bits -> exact out [m][n]."""
    out = E.gemv(x_rows, w_logical)
    return {
        "name": name, "note": note,
        "m": len(x_rows), "k": len(x_rows[0]) if x_rows else 0, "n": len(w_logical),
        "x": [f32hex(r) for r in x_rows],
        "w_nk": [hx(r, 4) for r in w_logical],
        "out": [f32hex(r) for r in out],
    }


def main():
    cases = []
    # --- jit.rs:30204-30243: m=3, k=5, n=4; a[i] = i*0.5 - 3, w[i] = trunc(i*0.25 - 2)
    m, k, n = 3, 5, 4
    a = [f32(f32(i) * f32(0.5) - f32(3.0)) for i in range(m * k)]
    wb = [trunc_bf16(f32(f32(i) * f32(0.25) - f32(2.0))) for i in range(k * n)]  # [k, n]
    x_rows = [a[r * k:(r + 1) * k] for r in range(m)]
    w_nk = [[wb[kk * n + j] for kk in range(k)] for j in range(n)]
    cases.append(gemv_case("jit_bf16_matmul_m3k5n4", x_rows, w_nk,
                           "compiler/src/jit.rs:30204-30243 inputs; exact fma chain"))
    # --- jit.rs:42643-42655: [1,2] ones @ bf16 [2,3] ones -> [2,2,2], sum 6
    cases.append(gemv_case("jit_bf16_field_matmul_ones", [[1.0, 1.0]], [[0x3F80] * 2] * 3,
                           "compiler/src/jit.rs:42643-42655: sum(x @ w) == 6"))
    # --- tools/jit_probes.py:932: 1x4 @ 4x1 ones -> 4
    cases.append(gemv_case("probe_matmul_1xN_Nx1", [[1.0] * 4], [[0x3F80] * 4],
                           "tools/jit_probes.py:932: (a@b)[0,0] == 4"))

    rng = np.random.Generator(np.random.PCG64(20261201))
    # --- random small: products are not exact in binary32 (separates fused from unfused)
    m, k, n = 3, 67, 11
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = ((rng.standard_normal((n, k)).astype(np.float32).view(np.uint32) + 0x7FFF) >> 16).astype(np.uint16)
    cases.append(gemv_case("random_m3k67n11", x.tolist(), w.tolist(),
                           "seeded N(0,1); exact fma chain"))

    # --- edge cases: NaN/inf/signed zeros/subnormals/1e-38
    tiny = f32(1e-38)
    xr = [1.5, -2.0, 0.0, -0.0, tiny, -tiny, 3.0, 1e-30, -0.5]
    k = len(xr)
    W = []
    W.append([0x3F80] * k)                                  # plain sum
    W.append([0x7F80] + [0x3F80] * (k - 1))                  # +inf * 1.5 -> +inf
    W.append([0x3F80, 0x3F80, 0x7F80] + [0] * (k - 3))       # +inf * +0 -> NaN
    W.append([0, 0, 0, 0, 0x7F80, 0, 0, 0, 0])               # +inf * 1e-38 -> +inf (no FTZ)
    W.append([0, 0, 0, 0, 0, 0xFF80, 0, 0, 0])               # -inf * -1e-38 -> +inf
    W.append([0x7F80, 0x7F80, 0, 0, 0, 0, 0, 0, 0])          # +inf + -inf -> NaN
    W.append([0x7FC0] + [0] * (k - 1))                       # NaN weight
    W.append([0x0000, 0x8000] * 4 + [0x8000])               # exact zero products -> +0
    W.append([0x8000] * k)                                  # all -0 weights -> +0
    W.append([0x0001, 0x807F, 0x0040, 0x8001, 0x0001, 0x0002, 0x0003, 0x0004, 0x0005])  # subnormals
    W.append([0x3F80, 0x3F80] + [0] * (k - 2))              # 1.5 - 2 = -0.5
    cases.append(gemv_case("edge_nan_inf_zero_subnormal", [xr], W,
                           "IEEE edge cases; exact fma chain"))

    # --- underflow: the sign of a zero result depends on the chain order
    # x = 1e-38 (subnormal), w = -/+ smallest bf16 subnormal: products ~1e-78 underflow
    xu = [tiny, tiny, tiny]
    Wu = [[0x8001, 0x0000, 0x0000],   # -tiny, +0, +0   -> -0 then -0 + +0 = +0
          [0x8001, 0x8000, 0x8000],   # -tiny, -0, -0   -> -0 stays -0
          [0x0000, 0x0000, 0x8001],   # last product underflows negative -> -0
          [0x8001, 0x0001, 0x8000]]   # -0 then +tiny -> +0, then -0 product keeps +0
    cases.append(gemv_case("underflow_signed_zero", [xu], Wu,
                           "zero results whose sign the chain order decides"))

    # --- every product an exact -0: the +0 seed decides (+0 + -0 = +0)
    xp = [1.0, 2.0, 0.5, 3.0]
    Wz = [[0x8000] * 4,                 # positive x * -0 -> all products -0
          [0x0000] * 4]                 # positive x * +0 -> all products +0
    cases.append(gemv_case("negative_zero_products", [xp, [-v for v in xp]], Wz,
                           "chains of exact -0 products start from +0 and stay +0"))

    # --- widen KAT (jit.rs:30171-30178) and transpose KAT (jit.rs:30249-30263)
    widen_in = [0x0000, 0x3F80, 0xBF80, 0x4000, 0x4049]
    widen_out = [0x00000000, 0x3F800000, 0xBF800000, 0x40000000, 0x40490000]
    tm, tn = 2, 3
    tsrc = [(0x3F00 + i * 0x80) & 0xFFFF for i in range(tm * tn)]
    tdst = [tsrc[i * tn + j] for j in range(tn) for i in range(tm)]

    doc = {
        "generator": "tests/golden/make_golden.py",
        "widen": {"in": hx(widen_in, 4), "out": hx(widen_out, 8),
                  "source": "compiler/src/jit.rs:30171-30178"},
        "truncate": {"in": f32hex([1.0, -1.0, 2.0, 3.140625, 1.0 + 2 ** -8, -0.0]),
                     "out": hx([0x3F80, 0xBF80, 0x4000, 0x4049, 0x3F80, 0x8000], 4),
                     "source": "compiler/src/jit.rs:29781-29792 (bits >> 16)"},
        "transpose": {"m": tm, "n": tn, "in": hx(tsrc, 4), "out": hx(tdst, 4),
                      "source": "compiler/src/jit.rs:30249-30263"},
        "gemv": cases,
    }
    out = HERE / "golden_vectors.json"
    out.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {out} ({len(cases)} GEMV cases)")


if __name__ == "__main__":
    main()
