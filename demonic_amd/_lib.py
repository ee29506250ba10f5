"""ctypes binding of libdmc_hip.so (declarations in include/dmc_hip.h).

The library is loaded from demonic_amd/lib/ only; if it is missing this module
raises BackendMissing with the build command.  There is no fallback: every
GEMV entry runs the gfx950 kernels or fails.
"""
from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "libdmc_hip.so"

i32, i64, f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_float
cstr = ctypes.c_char_p

# name -> (restype, argtypes); one line per declaration in include/dmc_hip.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "dmc_matmul_bf16_gpu": (None, [i64] * 6),
    "dmc_matmul_bf16_gpu_batched": (None, [i64] * 9),
    "dmc_matmul_bf16_gpu_batched_deferred": (None, [i64] * 9),
    "dmc_matmul_bf16_gpu_flush": (None, []),
    "dmc_matmul_bf16_gpu_t": (None, [i64] * 6),
    "dmc_matmul_bf16_gpu_try": (i32, [i64] * 6),
    "dmc_matmul_bf16_gpu_t_try": (i32, [i64] * 6),
    "dmc_matmul_bf16_gpu_batched_try": (i32, [i64] * 9),
    "dmc_matmul_bf16_gpu_batched_deferred_try": (i32, [i64] * 9),
    "dmc_matmul_bf16_gpu_flush_try": (i32, []),
    "dmc_matmul_f32_gpu": (None, [i64] * 6),
    "dmc_matmul_f32_gpu_try": (i32, [i64] * 6),
    "dmc_hip_f32_selected": (i32, [i32, i32, i64, i64, i64]),
    "dmc_hip_gemv_f32_rd": (i32, [i64] * 6),
    "dmc_hip_plan_f32": (i32, [i64, i64, i64, i64, i64, ctypes.POINTER(i64)]),
    "dmc_hip_available": (i32, []),
    "dmc_hip_gemv_selected": (i32, [i32, i32, i64, i64, i64]),
    "dmc_hip_last_error": (cstr, []),
    "dmc_hip_region_alloc": (i64, [i64]),
    "dmc_hip_region_free": (i32, [i64]),
    "dmc_hip_upload": (i32, [i64, i64, i64]),
    "dmc_hip_download": (i32, [i64, i64, i64]),
    "dmc_hip_copy_device": (i32, [i64, i64, i64]),
    "dmc_hip_register_weight": (i64, [i64, i64]),
    "dmc_hip_release_weights": (i32, []),
    "dmc_hip_resident_count": (i64, []),
    "dmc_hip_resident_bytes": (i64, []),
    "dmc_hip_gemv_cs": (i32, [i64] * 9),
    "dmc_hip_gemv_rd": (i32, [i64] * 6),
    "dmc_hip_gemv_cs_noalloc": (i32, [i64] * 9),
    "dmc_hip_synchronize": (i32, []),
    "dmc_hip_probe_read": (i32, [i64, i64]),
    "dmc_hip_gemv_rd_grouped": (i32, [i64, ctypes.POINTER(i64), ctypes.POINTER(i64),
                                      ctypes.POINTER(i64), ctypes.POINTER(i64), i64, i64]),
    "dmc_hip_fill_counter_bf16": (i32, [i64, i64, i64, ctypes.c_uint64, i64]),
    "dmc_hip_bf16_upconvert": (i32, [i64, i64, i64]),
    "dmc_hip_f32_to_bf16": (i32, [i64, i64, i64]),
    "dmc_hip_bf16_transpose_2d": (i32, [i64, i64, i64, i64]),
    "dmc_hip_f16_upconvert": (i32, [i64, i64, i64]),
    "dmc_hip_vault_load_npz": (i64, [cstr, cstr, i64, i64, i64]),
    "dmc_hip_npz_locate": (i32, [cstr, cstr, ctypes.POINTER(i64)]),
    "dmc_hip_plan": (i32, [i32, i64, i64, i64, i64, i64, i64, i64, ctypes.POINTER(i64)]),
    "dmc_hip_capture_begin": (i32, []),
    "dmc_hip_capture_end": (i64, []),
    "dmc_hip_graph_launch": (i32, [i64]),
    "dmc_hip_graph_destroy": (i32, [i64]),
    "dmc_hip_event_create": (i64, []),
    "dmc_hip_event_record": (i32, [i64]),
    "dmc_hip_event_synchronize": (i32, [i64]),
    "dmc_hip_event_elapsed_ms": (f32, [i64, i64]),
    "dmc_hip_event_destroy": (i32, [i64]),
    "dmc_hip_device_cus": (i32, []),
    "dmc_hip_device_arch": (cstr, []),
}


class BackendMissing(ImportError):
    """libdmc_hip.so is not built (or cannot be loaded)."""


class HipError(RuntimeError):
    """A libdmc_hip entry returned an error code."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"dmc_hip error {code}: {msg}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and declare the library once per process."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise BackendMissing(
                f"{LIB_PATH} is not built; run `python -m demonic_amd.build` "
                "(or __graft_entry__.build())")
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as e:
            raise BackendMissing(f"cannot load {LIB_PATH}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int) -> None:
    """Raise HipError for a negative return code."""
    if rc < 0:
        lib = load()
        raise HipError(rc, (lib.dmc_hip_last_error() or b"").decode(errors="replace"))
