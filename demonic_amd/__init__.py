"""demonic_amd -- MI355X (gfx950) bf16 GEMV backend for demoniC's `@` operator.

Python mirror of the C ABI in include/dmc_hip.h.  The functions keep the names
and argument meaning of the reference's Metal backend (compiler/src/gpu.rs:
400-474): `matmul_bf16_gpu` is dmc_matmul_bf16_gpu, `..._batched`,
`..._batched_deferred` and `flush` likewise, plus the MI355X additions
(transposed-RHS form, device regions, device-pointer GEMVs, events).

Host-pointer calls take NumPy arrays: activations float32, weights uint16
holding bf16 bit patterns, all C-contiguous.  Nothing here computes on the
CPU; if libdmc_hip.so is missing, every call raises BackendMissing.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import BackendMissing, HipError

__all__ = [
    "BackendMissing", "HipError", "available", "gemv_selected", "MIN_MACS",
    "matmul_bf16_gpu", "matmul_bf16_gpu_t", "matmul_bf16_gpu_batched",
    "matmul_bf16_gpu_batched_deferred", "flush", "DeviceBuffer", "gemv_cs", "gemv_rd",
    "synchronize", "probe_read", "gemv_rd_grouped", "fill_counter_bf16", "Graph", "Event", "plan", "register_weight", "release_weights",
    "resident_count", "resident_bytes", "device_info", "vault_load_npz", "npz_locate", "f16_upconvert",
]

MIN_MACS = 1 << 14  # DMC_HIP_MIN_MACS in include/dmc_hip.h


def _arr(a: np.ndarray, dtype, name: str) -> np.ndarray:
    if not isinstance(a, np.ndarray):
        raise TypeError(f"{name} must be a numpy array")
    if a.dtype != dtype:
        raise TypeError(f"{name} must be {np.dtype(dtype).name}, got {a.dtype}")
    if not a.flags.c_contiguous:
        raise ValueError(f"{name} must be C-contiguous")
    return a


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data if a.size else 0


def available() -> bool:
    """True when a gfx950 device is usable (cf. blas_gemm_available, jit.rs:29359)."""
    return bool(_lib.load().dmc_hip_available())


def gemv_selected(hip_on: bool, deterministic_depth: int, m: int, k: int, n: int) -> bool:
    """Route predicate, shaped like blas_gemm_selected (jit.rs:29346-29351)."""
    return bool(_lib.load().dmc_hip_gemv_selected(int(hip_on), deterministic_depth, m, k, n))


# Deferred outputs must stay alive until materialized; hold them here.
_pending_refs: list[np.ndarray] = []


def _dims2(x: np.ndarray) -> tuple[int, int]:
    if x.ndim == 1:
        return 1, x.shape[0]
    if x.ndim == 2:
        return x.shape
    raise ValueError("activation must be rank 1 or 2")


def matmul_bf16_gpu(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """out[m,n] = x[m,k] @ bf16(w[k,n]) -- dmc_matmul_bf16_gpu (gpu.rs:400-409)."""
    x = _arr(x, np.float32, "x")
    w = _arr(w, np.uint16, "w")
    m, k = _dims2(x)
    if w.ndim != 2 or w.shape[0] != k:
        raise ValueError(f"shape mismatch: x {x.shape} @ w {w.shape}")
    n = w.shape[1]
    out = np.empty((m, n), np.float32)
    _lib.load().dmc_matmul_bf16_gpu(_ptr(x), _ptr(w), _ptr(out), m, k, n)
    _pending_refs.clear()
    return out


def matmul_bf16_gpu_t(x: np.ndarray, w_nk: np.ndarray) -> np.ndarray:
    """out[m,n] = sum_k x[m,k] * bf16(w_nk[n,k]) -- `x @ W'` without the transpose."""
    x = _arr(x, np.float32, "x")
    w_nk = _arr(w_nk, np.uint16, "w_nk")
    m, k = _dims2(x)
    if w_nk.ndim != 2 or w_nk.shape[1] != k:
        raise ValueError(f"shape mismatch: x {x.shape} @ w_nk' {w_nk.shape}")
    n = w_nk.shape[0]
    out = np.empty((m, n), np.float32)
    _lib.load().dmc_matmul_bf16_gpu_t(_ptr(x), _ptr(w_nk), _ptr(out), m, k, n)
    _pending_refs.clear()
    return out


def _f32_operands(l: np.ndarray, r: np.ndarray):
    l = _arr(l, np.float32, "l")
    r = _arr(r, np.float32, "r")
    m, k = _dims2(l)
    if r.ndim == 1:
        r = r.reshape(-1, 1)
    if r.ndim != 2 or r.shape[0] != k:
        raise ValueError(f"shape mismatch: l {l.shape} @ r {r.shape}")
    return l, r, m, k, r.shape[1]


def matmul_f32_gpu(l: np.ndarray, r: np.ndarray) -> np.ndarray:
    """out[m,n] = l[m,k] @ r[k,n], all f32 -- dmc_matmul_f32_gpu, the device
    route of the reference's f32 `@` (jit.rs:20806-20831) on GEMV shapes."""
    l, r, m, k, n = _f32_operands(l, r)
    out = np.empty((m, n), np.float32)
    _lib.load().dmc_matmul_f32_gpu(_ptr(l), _ptr(r), _ptr(out), m, k, n)
    return out


def matmul_f32_gpu_try(l: np.ndarray, r: np.ndarray) -> tuple[int, np.ndarray]:
    """dmc_matmul_f32_gpu_try: (return code, out); out is untouched (zeros) on failure."""
    l, r, m, k, n = _f32_operands(l, r)
    out = np.zeros((m, n), np.float32)
    rc = _lib.load().dmc_matmul_f32_gpu_try(_ptr(l), _ptr(r), _ptr(out), m, k, n)
    return int(rc), out


def f32_selected(hip_on: bool, deterministic_depth: int, m: int, k: int, n: int) -> bool:
    """Route predicate of the f32 device route (dmc_hip_f32_selected)."""
    return bool(_lib.load().dmc_hip_f32_selected(int(hip_on), deterministic_depth, m, k, n))


def _check_batched(x, w, out, m, k, n, batch, ls, rs):
    x = _arr(x, np.float32, "x")
    w = _arr(w, np.uint16, "w")
    out = _arr(out, np.float32, "out")
    if min(m, k, n, batch, ls, rs) < 0:
        raise ValueError("negative size or stride")
    if batch and m and n:
        if x.size < (batch - 1) * ls + m * k:
            raise ValueError("x too small for batch/ls")
        if w.size < (batch - 1) * rs + k * n:
            raise ValueError("w too small for batch/rs")
        if out.size < batch * m * n:
            raise ValueError("out too small")
    return x, w, out


def matmul_bf16_gpu_batched(x, w, m, k, n, batch, ls, rs, out=None) -> np.ndarray:
    """dmc_matmul_bf16_gpu_batched (gpu.rs:410-437): slice z reads x[z*ls:], w[z*rs:]."""
    if out is None:
        out = np.empty(batch * m * n, np.float32)
    x, w, out = _check_batched(x, w, out, m, k, n, batch, ls, rs)
    _lib.load().dmc_matmul_bf16_gpu_batched(_ptr(x), _ptr(w), _ptr(out), m, k, n, batch, ls, rs)
    _pending_refs.clear()
    return out


def matmul_bf16_gpu_batched_deferred(x, w, out, m, k, n, batch, ls, rs) -> None:
    """dmc_matmul_bf16_gpu_batched_deferred (gpu.rs:439-466): `out` is written by
    the next synchronous call or flush(); it is kept alive until then."""
    x, w, out = _check_batched(x, w, out, m, k, n, batch, ls, rs)
    _lib.load().dmc_matmul_bf16_gpu_batched_deferred(
        _ptr(x), _ptr(w), _ptr(out), m, k, n, batch, ls, rs)
    _pending_refs.append(out)


def flush() -> None:
    """dmc_matmul_bf16_gpu_flush (gpu.rs:468-474)."""
    _lib.load().dmc_matmul_bf16_gpu_flush()
    _pending_refs.clear()


# ---- device regions and device-pointer GEMVs -------------------------------------

class DeviceBuffer:
    """A hipMalloc-backed HBM region (dmc_hip_region_alloc)."""

    def __init__(self, nbytes: int):
        lib = _lib.load()
        self.nbytes = int(nbytes)
        self.addr = lib.dmc_hip_region_alloc(self.nbytes)
        if not self.addr:
            _lib.check(-3)

    @classmethod
    def adopt(cls, addr: int, nbytes: int) -> "DeviceBuffer":
        """Take ownership of a region the library allocated (freed by free())."""
        buf = cls.__new__(cls)
        buf.addr, buf.nbytes = int(addr), int(nbytes)
        return buf

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(max(a.nbytes, 1))
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload beyond region")
        _lib.check(_lib.load().dmc_hip_upload(self.addr + offset, _ptr(a), a.nbytes))

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download beyond region")
        _lib.check(_lib.load().dmc_hip_download(_ptr(out), self.addr + offset, out.nbytes))
        return out

    def copy_from(self, src: "DeviceBuffer", nbytes: int | None = None) -> None:
        n = src.nbytes if nbytes is None else nbytes
        if n > self.nbytes or n > src.nbytes:
            raise ValueError("copy beyond region")
        _lib.check(_lib.load().dmc_hip_copy_device(self.addr, src.addr, n))

    def free(self) -> None:
        if self.addr:
            _lib.check(_lib.load().dmc_hip_region_free(self.addr))
            self.addr = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


def _addr(b) -> int:
    return b.addr if isinstance(b, DeviceBuffer) else int(b)


def gemv_cs(x, w, y, m: int, k: int, n: int, batch: int = 1, ls: int = 0, rs: int = 0) -> None:
    """Enqueue y[z] = x[z] @ bf16(w[z]) on device regions (w [k,n] per slice)."""
    _lib.check(_lib.load().dmc_hip_gemv_cs(_addr(x), _addr(w), _addr(y), m, k, n, batch, ls, rs))


def gemv_rd(x, w, y, m: int, k: int, n: int) -> None:
    """Enqueue y = x @ bf16(w)' on device regions (w [n,k], the row-dot layout)."""
    _lib.check(_lib.load().dmc_hip_gemv_rd(_addr(x), _addr(w), _addr(y), m, k, n))


def gemv_f32_rd(x, w, y, m: int, k: int, n: int) -> None:
    """Enqueue y = x @ w' on device regions, f32 weights (w [n,k])."""
    _lib.check(_lib.load().dmc_hip_gemv_f32_rd(_addr(x), _addr(w), _addr(y), m, k, n))


def gemv_rd_grouped(xs, ws, ys, ns, m: int, k: int) -> None:
    """Enqueue y_i = x_i @ bf16(w_i)' for independent problems sharing m and k
    (w_i [n_i, k] row-dot weights), one launch per 8 problems."""
    cnt = len(ns)
    if not (len(xs) == len(ws) == len(ys) == cnt):
        raise ValueError("xs, ws, ys and ns must have the same length")
    arr = lambda v: (ctypes.c_int64 * max(cnt, 1))(*[int(a) for a in v])  # noqa: E731
    _lib.check(_lib.load().dmc_hip_gemv_rd_grouped(
        cnt, arr(_addr(b) for b in xs), arr(_addr(b) for b in ws), arr(_addr(b) for b in ys),
        arr(ns), m, k))


def fill_counter_bf16(dst, count: int, key: int, table, offset: int = 0) -> None:
    """Fill a device region with counter-generated bf16 bits (the generator of
    workloads.counter_bf16, run in HBM); `table` is a device copy of the
    65,536-entry table."""
    _lib.check(_lib.load().dmc_hip_fill_counter_bf16(_addr(dst), count, offset, key & ((1 << 64) - 1),
                                                     _addr(table)))


def bf16_upconvert(src, dst, n: int) -> None:
    """Enqueue dst f32[n] = widen(src bf16[n]) (dmc_bf16_upconvert, jit.rs:29760)."""
    _lib.check(_lib.load().dmc_hip_bf16_upconvert(_addr(src), _addr(dst), n))


def f32_to_bf16(src, dst, n: int) -> None:
    """Enqueue dst bf16[n] = src f32 bits >> 16 (dmc_f32_to_bf16, jit.rs:29783)."""
    _lib.check(_lib.load().dmc_hip_f32_to_bf16(_addr(src), _addr(dst), n))


def f16_upconvert(src, dst, n: int) -> None:
    """Enqueue dst f32[n] = the IEEE f16 patterns src[n] widened exactly
    (f16_bits_to_f32, jit.rs:29231-29257)."""
    _lib.check(_lib.load().dmc_hip_f16_upconvert(_addr(src), _addr(dst), n))


# ---- weight ingress ---------------------------------------------------------------

# vault.load_npz dtypes: (on-disk element bytes, convert) as the JIT lowers
# them (jit.rs:12671-12681); bf16 stays 2-byte (the Bf16Tensor route).
NPZ_DTYPES = {"f32": (4, 0), "f64": (8, 0), "i32": (4, 0), "i64": (8, 0), "bf16": (2, 0),
              "f16": (2, 2), "bool": (1, 0)}


def vault_load_npz(path, key: str, numel: int, elem_bytes: int = 2, convert: int = 0) -> DeviceBuffer:
    """dmc_hip_vault_load_npz: array `key` of the .npz at `path` in a new
    device region (numel * elem_bytes bytes, numel * 4 when convert widens,
    plus 16 zero bytes of padding).  Raises HipError where the reference's
    dmc_vault_load_npz (jit.rs:29836-29926) returns 0."""
    lib = _lib.load()
    addr = lib.dmc_hip_vault_load_npz(str(path).encode(), key.encode(), numel, elem_bytes, convert)
    if not addr:
        raise HipError(-5, lib.dmc_hip_last_error().decode())
    out_bytes = numel * (4 if convert else elem_bytes)
    return DeviceBuffer.adopt(addr, out_bytes + 16)


def npz_locate(path, key: str) -> dict:
    """Where dmc_hip_vault_load_npz finds `key` (no device needed)."""
    info = (ctypes.c_int64 * 8)()
    _lib.check(_lib.load().dmc_hip_npz_locate(str(path).encode(), key.encode(), info))
    names = ("bare", "method", "compressed", "uncompressed", "data_pos", "npy_major", "npy_data_offset", "crc")
    return dict(zip(names, [int(v) for v in info]))


def bf16_transpose_2d(src, dst, m: int, n: int) -> None:
    """Enqueue dst [n, m] = src [m, n]^T on bf16 bit patterns
    (dmc_bf16_transpose_2d, jit.rs:29801)."""
    _lib.check(_lib.load().dmc_hip_bf16_transpose_2d(_addr(src), _addr(dst), m, n))


def synchronize() -> None:
    _lib.check(_lib.load().dmc_hip_synchronize())


def probe_read(buf, nbytes: int | None = None) -> None:
    """Enqueue a read-only pass over a device region (the stream-read ceiling
    probe); nbytes=0 enqueues an empty launch (the dispatch floor)."""
    n = buf.nbytes if nbytes is None else int(nbytes)
    _lib.check(_lib.load().dmc_hip_probe_read(_addr(buf) if n else 0, n))


class Graph:
    """A captured sequence of device-pointer GEMVs, replayed with one call.

        with Graph() as g:      # capture
            gemv_rd(...); gemv_rd_grouped(...)
        g.launch()              # replay on the library stream
    """

    def __init__(self):
        self.exec = 0

    def __enter__(self):
        _lib.check(_lib.load().dmc_hip_capture_begin())
        return self

    def __exit__(self, exc_type, *exc):
        ex = _lib.load().dmc_hip_capture_end()
        if exc_type is None:
            if not ex:
                _lib.check(-4)
            self.exec = ex
        elif ex:
            _lib.load().dmc_hip_graph_destroy(ex)
        return False

    def launch(self) -> None:
        _lib.check(_lib.load().dmc_hip_graph_launch(self.exec))

    def destroy(self) -> None:
        if self.exec:
            _lib.check(_lib.load().dmc_hip_graph_destroy(self.exec))
            self.exec = 0


class Event:
    """A HIP event recorded on the library stream."""

    def __init__(self):
        self.ev = _lib.load().dmc_hip_event_create()
        if not self.ev:
            _lib.check(-4)

    def record(self) -> None:
        _lib.check(_lib.load().dmc_hip_event_record(self.ev))

    def synchronize(self) -> None:
        _lib.check(_lib.load().dmc_hip_event_synchronize(self.ev))

    def elapsed_ms(self, end: "Event") -> float:
        ms = _lib.load().dmc_hip_event_elapsed_ms(self.ev, end.ev)
        if ms < 0:
            raise HipError(-4, "hipEventElapsedTime failed")
        return ms

    def __del__(self):
        try:
            if self.ev and _lib._lib is not None:
                _lib._lib.dmc_hip_event_destroy(self.ev)
        except Exception:
            pass


@dataclass
class Plan:
    vec: int
    rows_or_rw: int        # rd: weight rows per register buffer; cs: the general kernel's k rows
                           # per wave-wide load (> 0), or the streaming kernel's -row groups (<= 0)
    mt: int
    grid_x: int
    slices: int            # cs: k slices; rd: 8-element k vectors per lane (0 = general kernel)
    workspace_bytes: int
    waves: int
    rows_per_group: int    # rd: weight rows per workgroup; cs: k rows per workgroup
                           # (streaming kernel) or columns per workgroup (general)


def plan(layout: str, m: int, k: int, n: int, batch: int = 1, rs: int = 0,
         x_addr: int = 0, w_addr: int = 0) -> Plan:
    """Launch plan for layout 'rd' or 'cs' (pure host computation)."""
    out = (ctypes.c_int64 * 8)()
    _lib.check(_lib.load().dmc_hip_plan(int(layout == "rd"), x_addr, w_addr, m, k, n, batch, rs, out))
    return Plan(*[int(v) for v in out])


@dataclass
class PlanF32:
    kvec: int              # 4-element k vectors per lane (0 = general kernel)
    rows: int              # weight rows per register buffer
    mt: int                # activation rows per workgroup
    grid_x: int
    grid_y: int
    waves: int
    rows_per_group: int    # weight rows per workgroup


def plan_f32(m: int, k: int, n: int, x_addr: int = 0, w_addr: int = 0) -> PlanF32:
    """Launch plan of the f32 row-dot GEMV (pure host computation)."""
    out = (ctypes.c_int64 * 8)()
    _lib.check(_lib.load().dmc_hip_plan_f32(x_addr, w_addr, m, k, n, out))
    return PlanF32(*[int(v) for v in out[:7]])


def register_weight(w: np.ndarray) -> int:
    """Make a host weight resident now; returns its device address."""
    w = np.ascontiguousarray(w)
    d = _lib.load().dmc_hip_register_weight(_ptr(w), w.nbytes)
    if not d:
        _lib.check(-3)
    return d


def release_weights() -> None:
    _lib.check(_lib.load().dmc_hip_release_weights())


def resident_count() -> int:
    return int(_lib.load().dmc_hip_resident_count())


def resident_bytes() -> int:
    return int(_lib.load().dmc_hip_resident_bytes())


def device_info() -> dict:
    lib = _lib.load()
    return {"arch": (lib.dmc_hip_device_arch() or b"").decode(), "cus": int(lib.dmc_hip_device_cus())}
