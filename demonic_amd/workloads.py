"""Seeded synthetic inputs for the five GEMV configurations.

Weights are bf16 bit patterns (uint16); activations are float32.  Logical
weights are indexed w[n, k] (output n, reduction k).  A row-dot (RD) weight is
stored as that [N, K] array; a column-stream (CS) weight is its transpose, stored
[K, N].  Both layouts of one logical weight give the same reference output.

Generator (dense configs): numpy Generator(PCG64(seed)); W drawn first as
scale * standard_normal(float32) and rounded to nearest-even bf16, then x as
standard_normal(float32).

Counter generator (the 32-layer sweep, ~14 GB): element i of tensor t is
TABLE[splitmix64(seed, t, i) >> 48], TABLE being the 65,536-entry bf16
inverse-normal table below; the device fills HBM with the same bits.
"""
from __future__ import annotations

import numpy as np

# Llama-3-8B decode projections (per layer): (name, N, K), row-dot layout.
LLAMA3_8B_LAYER = (
    ("q", 4096, 4096),
    ("k", 1024, 4096),
    ("v", 1024, 4096),
    ("o", 4096, 4096),
    ("gate", 14336, 4096),
    ("up", 14336, 4096),
    ("down", 4096, 14336),
)
LLAMA3_8B_LAYERS = 32
LM_HEAD = (128256, 4096)


def bf16_rne(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """Exact widen, bits << 16 (compiler/src/jit.rs:29225-29227)."""
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dense(n: int, k: int, seed: int, scale: float = 0.02, m: int = 1):
    """Logical W[n,k] ~ N(0, scale) in bf16 and x[m,k] ~ N(0,1) f32."""
    rng = np.random.Generator(np.random.PCG64(seed))
    w = bf16_rne(np.float32(scale) * rng.standard_normal((n, k), dtype=np.float32))
    x = rng.standard_normal((m, k), dtype=np.float32)
    return w, x


def c1(seed: int = 0):
    """C1: single GEMV, W [4096,4096] ~N(0,0.02), x [4096] ~N(0,1)."""
    return dense(4096, 4096, seed)


def c2(seed: int = 0):
    """C2: Llama-3-8B FFN decode shapes: up/gate W [14336,4096], down W [4096,14336]."""
    return {"up": dense(14336, 4096, seed), "down": dense(4096, 14336, seed + 1)}


def c4(m: int, seed: int = 0):
    """C4: LM head W [128256,4096] ~N(0,0.02), X [m,4096] ~N(0,1)."""
    return dense(LM_HEAD[0], LM_HEAD[1], seed, m=m)


# ---- C5: numerics and edge shapes -------------------------------------------------

C5_SHAPES = ((11008, 4097), (4097, 11008))


def c5(n: int, k: int, seed: int = 0, m: int = 1):
    """C5 logical weight W[n,k] ~N(0,1) bf16 with 0.1% bf16 subnormals and
    seeded +-inf / NaN injections, and x with +0, -0 and +-1e-38 entries.

    Returns (w, x, rows) where rows names the output rows built to exercise a
    specific rule (each is also a plain output to compare):
      inf_pos     one +inf weight against a normal x            -> +inf
      inf_neg_x   -inf weight against a negative normal x        -> +inf
      inf_both    +inf and -inf weights, both against x > 0      -> NaN
      inf_zero    +inf weight where x = +0                       -> NaN
      inf_nzero   +inf weight where x = -0                       -> NaN
      inf_tiny    +inf weight where x = +1e-38 (f32 subnormal)   -> +inf
      inf_ntiny   -inf weight where x = -1e-38                   -> +inf
      nan_w       NaN weight                                     -> NaN
      zero_row    all weights +-0 (x finite)                     -> +0
      negzero_row all weights -0 (x finite)                      -> +0
      sub_row     every weight a bf16 subnormal                  -> tiny, finite
    """
    # one stream per shape: the two C5 weights must not share their bytes
    rng = np.random.Generator(np.random.PCG64([seed, n, k]))
    w = bf16_rne(rng.standard_normal((n, k), dtype=np.float32))
    # 0.1% subnormals: exponent 0, mantissa 1..127, random sign
    cnt = max(1, (n * k) // 1000)
    pos = rng.choice(n * k, size=cnt, replace=False)
    mant = rng.integers(1, 128, size=cnt, dtype=np.uint16)
    sign = rng.integers(0, 2, size=cnt, dtype=np.uint16) << 15
    w.reshape(-1)[pos] = sign | mant

    x = rng.standard_normal((m, k), dtype=np.float32)
    # ~1% each of +0, -0 and +-1e-38 (f32 subnormal), per activation row
    per = max(1, k // 100)
    tiny = np.float32(1e-38)
    for i in range(m):
        idx = rng.permutation(k)
        x[i, idx[:per]] = np.float32(0.0)
        x[i, idx[per:2 * per]] = np.float32(-0.0)
        t = idx[2 * per:3 * per]
        x[i, t] = np.where(rng.integers(0, 2, size=t.size) == 0, tiny, -tiny)

    x0 = x[0]
    pinf, ninf, qnan = np.uint16(0x7F80), np.uint16(0xFF80), np.uint16(0x7FC0)
    normal_pos = np.flatnonzero((np.abs(x0) > 1e-3) & (x0 > 0))
    normal_neg = np.flatnonzero((np.abs(x0) > 1e-3) & (x0 < 0))
    zero_p = np.flatnonzero((x0 == 0) & ~np.signbit(x0))
    zero_n = np.flatnonzero((x0 == 0) & np.signbit(x0))
    tiny_p = np.flatnonzero(x0 == tiny)
    tiny_n = np.flatnonzero(x0 == -tiny)

    rows = {}
    names = ["inf_pos", "inf_neg_x", "inf_both", "inf_zero", "inf_nzero", "inf_tiny",
             "inf_ntiny", "nan_w", "zero_row", "negzero_row", "sub_row"]
    chosen = rng.choice(n, size=len(names), replace=False)
    for name, r in zip(names, chosen):
        rows[name] = int(r)

    def pick(cands):
        return int(cands[rng.integers(0, cands.size)])

    w[rows["inf_pos"], pick(normal_pos)] = pinf
    w[rows["inf_neg_x"], pick(normal_neg)] = ninf
    kp = pick(normal_pos)
    w[rows["inf_both"], kp] = pinf
    w[rows["inf_both"], pick(np.setdiff1d(normal_pos, [kp]))] = ninf
    w[rows["inf_zero"], pick(zero_p)] = pinf
    w[rows["inf_nzero"], pick(zero_n)] = pinf
    w[rows["inf_tiny"], pick(tiny_p)] = pinf
    w[rows["inf_ntiny"], pick(tiny_n)] = ninf
    w[rows["nan_w"], rng.integers(0, k)] = qnan
    # exact-zero products only: the reference chain from +0 ends at +0
    w[rows["zero_row"], :] = rng.integers(0, 2, size=k).astype(np.uint16) << 15
    w[rows["negzero_row"], :] = np.uint16(0x8000)
    w[rows["sub_row"], :] = (rng.integers(0, 2, size=k).astype(np.uint16) << 15) | \
        rng.integers(1, 128, size=k, dtype=np.uint16)
    # 8 more random injections of each of +inf, -inf, NaN, off the named rows
    free_rows = np.setdiff1d(np.arange(n), chosen)
    for v in (pinf, ninf, qnan):
        rr = rng.choice(free_rows, size=8)
        kk = rng.integers(0, k, size=8)
        w[rr, kk] = v
    return w, x, rows


# ---- counter-based generator (device-fillable) --------------------------------------

_MASK = (1 << 64) - 1


def _splitmix64_np(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64)
    z = z + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def counter_seed(seed: int, tensor: int) -> int:
    """Per-tensor 64-bit stream key."""
    return (seed * 0xD1B54A32D192ED03 + tensor * 0x8CB92BA72F3D8DD7 + 0x2545F4914F6CDD1D) & _MASK


_TABLE_CACHE: dict[float, np.ndarray] = {}


def normal_table(scale: float) -> np.ndarray:
    """65,536-entry bf16 table: bf16_rne(scale * Phi^-1((u + 0.5) / 65536))."""
    t = _TABLE_CACHE.get(scale)
    if t is None:
        from scipy.special import ndtri
        u = (np.arange(65536, dtype=np.float64) + 0.5) / 65536.0
        t = bf16_rne((scale * ndtri(u)).astype(np.float32))
        _TABLE_CACHE[scale] = t
    return t


def counter_bf16(seed: int, tensor: int, count: int, offset: int = 0, scale: float = 0.02):
    """Elements [offset, offset+count) of counter-generated tensor `tensor`."""
    key = np.uint64(counter_seed(seed, tensor))
    idx = np.arange(offset, offset + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = _splitmix64_np(idx ^ key)
    return normal_table(scale)[(h >> np.uint64(48)).astype(np.int64)]


# ---- C3: the 32-layer decode sweep --------------------------------------------------

C3_SCALE = 0.02


def c3_tensor(layer: int, idx: int) -> int:
    """Counter-generator tensor id of projection idx (LLAMA3_8B_LAYER order) of a layer."""
    return layer * len(LLAMA3_8B_LAYER) + idx


def c3_x(layer: int, k: int, seed: int = 0) -> np.ndarray:
    """The layer's activation of length k (4096, or 14336 for down), ~N(0,1)."""
    return counter_f32_normal(seed, 1_000_000 + 2 * layer + (k != 4096), k)


def c3_rows(layer: int, idx: int, rows, seed: int = 0) -> np.ndarray:
    """Rows `rows` of projection idx of a layer, regenerated on the host
    (bit-identical to the device fill)."""
    _, n, k = LLAMA3_8B_LAYER[idx]
    return counter_rows(seed, c3_tensor(layer, idx), rows, k, C3_SCALE)


def counter_rows(seed: int, tensor: int, rows, k: int, scale: float = 0.02) -> np.ndarray:
    """Rows `rows` [len(rows), k] of a counter-generated [N, k] tensor."""
    out = np.empty((len(rows), k), np.uint16)
    for j, r in enumerate(rows):
        out[j] = counter_bf16(seed, tensor, k, offset=int(r) * k, scale=scale)
    return out


# ---- C4: the LM head at full size, generated in HBM ----------------------------------

C4_TENSOR = 900_000  # counter-generator tensor id of the full-size LM-head weight


def counter_f32_normal(seed: int, tensor: int, count: int) -> np.ndarray:
    """Activation vector for the sweep: N(0,1) float32 from PCG64(seed, tensor)."""
    rng = np.random.Generator(np.random.PCG64([seed, tensor]))
    return rng.standard_normal(count, dtype=np.float32)
