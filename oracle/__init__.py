"""ctypes binding of the CPU oracle (oracle/dmc_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker and the timed CPU baseline.  The
product package (demonic_amd) never imports it.

Build: `make -C oracle` (or demonic_amd.build), producing oracle/lib/*.so.
"""
from __future__ import annotations

import contextlib
import ctypes
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "lib" / "libdmc_oracle.so"
LIB_V3 = HERE / "lib" / "libdmc_oracle_v3.so"

MUTATIONS = {
    "drop_last_k": 1,
    "neg_zero_init": 2,
    "unfused": 3,
    "transposed_w": 4,
    "widen_shift": 5,
    "descending_k": 6,
}

_i64, _i32 = ctypes.c_int64, ctypes.c_int
_P = ctypes.c_void_p
_cache: dict[str, ctypes.CDLL] = {}


def load(variant: str = "port") -> ctypes.CDLL:
    """variant "port": scalar build like the reference's x86 build (the checker);
    "v3": the same source vectorized for x86-64-v3 (the strong CPU baseline)."""
    if variant in _cache:
        return _cache[variant]
    path = LIB if variant == "port" else LIB_V3
    if not path.exists():
        raise FileNotFoundError(f"{path} not built; run `make -C {HERE}`")
    lib = ctypes.CDLL(str(path))
    lib.oracle_bf16_to_f32.restype = ctypes.c_float
    lib.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    for name in ("oracle_bf16_upconvert", "oracle_f32_to_bf16_n"):
        getattr(lib, name).argtypes = [_P, _P, _i64]
    lib.oracle_bf16_transpose.argtypes = [_P, _P, _i64, _i64]
    lib.oracle_matmul_bf16.argtypes = [_P, _P, _P, _i64, _i64, _i64]
    lib.oracle_matmul_bf16_ex.argtypes = [_P, _P, _P, _i64, _i64, _i64, _i32]
    lib.oracle_matmul_bf16_t.restype = _i32
    lib.oracle_matmul_bf16_t.argtypes = [_P, _P, _P, _i64, _i64, _i64]
    lib.oracle_gemv_points.argtypes = [_P, _i64, _P, _i64, _i32, _i64, _P, _P, _i64, _P]
    lib.oracle_matmul_bf16_batched.argtypes = [_P, _P, _P, _i64, _i64, _i64, _i64, _i64]
    lib.oracle_matmul_f32.argtypes = [_P, _P, _P, _i64, _i64, _i64]
    lib.oracle_gemv_points_f32.argtypes = [_P, _i64, _P, _i64, _i64, _P, _P, _i64, _P]
    lib.oracle_matmul_threads.restype = _i32
    lib.oracle_matmul_threads.argtypes = [_i64, _i64, _i64]
    lib.oracle_gemv_ways.restype = _i32
    lib.oracle_gemv_ways.argtypes = [_i64, _i64]
    lib.oracle_set_mutation.argtypes = [_i32]
    lib.oracle_get_mutation.restype = _i32
    _cache[variant] = lib
    return lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def widen(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    load().oracle_bf16_upconvert(_p(h), _p(out), h.size)
    return out


def truncate(f) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    load().oracle_f32_to_bf16_n(_p(f), _p(out), f.size)
    return out


def transpose(w) -> np.ndarray:
    w = _c(w, np.uint16)
    m, n = w.shape
    out = np.empty((n, m), np.uint16)
    load().oracle_bf16_transpose(_p(w), _p(out), m, n)
    return out


def matmul_bf16(x, w_kn, workers: int = 0, variant: str = "port") -> np.ndarray:
    """Reference dmc_matmul_bf16: x[m,k] @ bf16(w[k,n]) (workers 0 = its policy)."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    w_kn = _c(w_kn, np.uint16)
    m, k = x.shape
    k2, n = w_kn.shape
    assert k == k2, (x.shape, w_kn.shape)
    out = np.empty((m, n), np.float32)
    load(variant).oracle_matmul_bf16_ex(_p(x), _p(w_kn), _p(out), m, k, n, workers)
    return out


def matmul_bf16_t(x, w_nk) -> np.ndarray:
    """Reference `x @ W'`: native-width transpose, then dmc_matmul_bf16."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    w_nk = _c(w_nk, np.uint16)
    m, k = x.shape
    n, k2 = w_nk.shape
    assert k == k2
    out = np.empty((m, n), np.float32)
    rc = load().oracle_matmul_bf16_t(_p(x), _p(w_nk), _p(out), m, k, n)
    if rc:
        raise MemoryError("oracle transpose buffer")
    return out


def gemv_points(x, w, layout: str, mi, ni) -> np.ndarray:
    """Closed form at selected outputs.  layout 'cs': w is [K,N]; 'rd': w is [N,K]."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    w = _c(w, np.uint16)
    mi = _c(mi, np.int64)
    ni = _c(ni, np.int64)
    assert mi.shape == ni.shape
    k = x.shape[1]
    ldw = w.shape[1]
    if layout == "cs":
        assert w.shape[0] == k
        lay = 0
    else:
        assert w.shape[1] == k
        lay = 1
    out = np.empty(mi.shape, np.float32)
    load().oracle_gemv_points(_p(x), x.shape[1], _p(w), ldw, lay, k, _p(mi), _p(ni), mi.size, _p(out))
    return out


def matmul_f32(l, r) -> np.ndarray:
    """Reference f32 `@` (dmc_matmul_par / scalar_matmul): l[m,k] @ r[k,n]."""
    l = _c(l, np.float32)
    if l.ndim == 1:
        l = l[None, :]
    r = _c(r, np.float32)
    if r.ndim == 1:
        r = r[:, None]
    m, k = l.shape
    k2, n = r.shape
    assert k == k2, (l.shape, r.shape)
    out = np.empty((m, n), np.float32)
    load().oracle_matmul_f32(_p(l), _p(r), _p(out), m, k, n)
    return out


def gemv_points_f32(x, w_nk, mi, ni) -> np.ndarray:
    """f32 closed form at outputs (mi[p], ni[p]) of x[m,k] @ w_nk[n,k]'."""
    x = _c(x, np.float32)
    if x.ndim == 1:
        x = x[None, :]
    w_nk = _c(w_nk, np.float32)
    mi = _c(mi, np.int64)
    ni = _c(ni, np.int64)
    k = x.shape[1]
    assert w_nk.shape[1] == k
    out = np.empty(mi.shape, np.float32)
    load().oracle_gemv_points_f32(_p(x), k, _p(w_nk), k, k, _p(mi), _p(ni), mi.size, _p(out))
    return out


def matmul_bf16_batched(x, w, k, n, batch, ls, rs) -> np.ndarray:
    """The Metal backend's batched CPU fallback (gpu.rs:366-391), m = 1."""
    x = _c(x, np.float32)
    w = _c(w, np.uint16)
    out = np.empty(batch * n, np.float32)
    load().oracle_matmul_bf16_batched(_p(x), _p(w), _p(out), k, n, batch, ls, rs)
    return out


def gemv_ways(k: int, n: int) -> int:
    return int(load().oracle_gemv_ways(k, n))


def matmul_threads(m: int, k: int, n: int) -> int:
    return int(load().oracle_matmul_threads(m, k, n))


@contextlib.contextmanager
def mutation(name: str):
    """Plant one mistake in the oracle for the duration of the block."""
    lib = load()
    lib.oracle_set_mutation(MUTATIONS[name])
    try:
        yield
    finally:
        lib.oracle_set_mutation(0)
