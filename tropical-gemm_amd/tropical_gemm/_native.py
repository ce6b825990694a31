"""ctypes binding of ``libtropical_gemm_hip.so`` (the C ABI in
``include/tropical_gemm_hip.h``).

This is the Python counterpart of what the reference's PyO3 module binds from
the Rust CUDA crate (``crates/tropical-gemm-python/src/lib.rs:1657-2601``).
There is no silent fallback: if the shared library is missing, every GPU entry
point raises ``RuntimeError`` naming the path it looked for.
"""
from __future__ import annotations

import ctypes
import os
import threading

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_PKG_DIR, "..", "libtropical_gemm_hip.so"))

# Status codes (tropical_gemm_hip.h); one per CudaError variant of the
# reference (crates/tropical-gemm-cuda/src/error.rs:8-29).
TG_OK = 0
TG_ERR_DRIVER = 1
TG_ERR_COMPILE = 2
TG_ERR_NO_DEVICE = 3
TG_ERR_DIMENSION_MISMATCH = 4
TG_ERR_KERNEL_NOT_FOUND = 5
TG_ERR_INVALID_ARGUMENT = 6
TG_ERR_UNSUPPORTED = 7

SEMIRING = {"maxplus": 0, "minplus": 1, "maxmul": 2}
DTYPE = {"f32": 0, "f64": 1, "i32": 2, "i64": 3}
LAYOUT = {"row": 0, "col": 1}

# Every symbol the header declares, with its ctypes signature.
_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
SIGNATURES = {
    "tg_version": ([], _i32),
    "tg_status_string": ([_i32], ctypes.c_char_p),
    "tg_last_error": ([], ctypes.c_char_p),
    "tg_device_count": ([ctypes.POINTER(_i32)], _i32),
    "tg_context_init": ([_i32], _i32),
    "tg_device_name": ([_i32, ctypes.c_char_p, _sz], _i32),
    "tg_malloc": ([_i32, ctypes.POINTER(_vp), _sz], _i32),
    "tg_free": ([_i32, _vp], _i32),
    "tg_memcpy_htod": ([_i32, _vp, _vp, _sz], _i32),
    "tg_memcpy_dtoh": ([_i32, _vp, _vp, _sz], _i32),
    "tg_memcpy_dtod": ([_i32, _vp, _vp, _sz, _vp], _i32),
    "tg_memset_zero": ([_i32, _vp, _sz, _vp], _i32),
    "tg_synchronize": ([_i32], _i32),
    "tg_stream_synchronize": ([_i32, _vp], _i32),
    "tg_kernel_timing_enable": ([_i32], _i32),
    "tg_kernel_timing_read": ([ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64)], _i32),
    "tg_gemm": ([_i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "tg_gemm_noalloc": ([_i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "tg_gemm_noalloc_bytes": ([_i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64], _sz),
    "tg_gemm_workspace_size": ([_i32, _i64, _i64, _i64, _i64, _i32], _sz),
    "tg_gemm_ws": ([_i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp],
                   _i32),
    "tg_gemm_plan": ([_i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                      _i64, _sz], ctypes.c_char_p),
    "tg_backward_plan": ([_i32, _i32, _i32, _i64, _i64, _i64, _i64], ctypes.c_char_p),
    "tg_gemm_strided_batched": ([_i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                 _i64, _i64, _i64, _i64, _vp], _i32),
    "tg_gemm_strided_batched_ws": ([_i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                    _i64, _i64, _i64, _i64, _vp, _sz, _vp], _i32),
    "tg_backward_a": ([_i32, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "tg_backward_b": ([_i32, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "tg_maxmul_backward_a": ([_i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "tg_maxmul_backward_b": ([_i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
    "tg_backward_a_strided_batched": ([_i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                       _i64, _i64, _i64, _i64, _vp], _i32),
    "tg_backward_b_strided_batched": ([_i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                       _i64, _i64, _i64, _i64, _vp], _i32),
    "tg_transpose": ([_i32, _i32, _vp, _vp, _i64, _i64, _i64, _vp], _i32),
}


class HipError(RuntimeError):
    """Error raised by the native library.  ``kind`` names the reference
    ``CudaError`` variant (Driver, Compile, NoDevice, DimensionMismatch,
    KernelNotFound) or InvalidArgument / Unsupported."""

    KINDS = {
        TG_ERR_DRIVER: "Driver",
        TG_ERR_COMPILE: "Compile",
        TG_ERR_NO_DEVICE: "NoDevice",
        TG_ERR_DIMENSION_MISMATCH: "DimensionMismatch",
        TG_ERR_KERNEL_NOT_FOUND: "KernelNotFound",
        TG_ERR_INVALID_ARGUMENT: "InvalidArgument",
        TG_ERR_UNSUPPORTED: "Unsupported",
    }

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = self.KINDS.get(status, "Unknown")
        super().__init__(f"{self.kind}: {message}")


_lib = None
_lock = threading.Lock()


def library_path() -> str:
    return LIB_PATH


def load():
    """Load the shared library once; raise if it is missing or incomplete."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"tropical_gemm native library not found at {LIB_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` or `make -C tropical-gemm_amd`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError if a declared symbol is missing
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def gemm_plan(semiring: str, dtype: str, m: int, n: int, k: int, with_argmax: bool = True,
              layout: str = "row", workspace_bytes: int | None = None, batch: int = 1,
              strides=(0, 0, 0), addresses=(256, 256, 256, 256)) -> str:
    """Name of the kernel path a product would run on (host logic only; the
    addresses stand for 16-byte aligned buffers and are never touched).
    workspace_bytes None: the full workspace, as tg_gemm allocates it."""
    lib = load()
    if workspace_bytes is None:
        workspace_bytes = lib.tg_gemm_workspace_size(DTYPE[dtype], batch, m, n, k, int(with_argmax))
    a, b, c, i = addresses
    return lib.tg_gemm_plan(SEMIRING[semiring], DTYPE[dtype], LAYOUT[layout], a, b, c,
                            i if with_argmax else None, batch, m, n, k, *strides,
                            workspace_bytes).decode()


def last_error() -> str:
    return load().tg_last_error().decode(errors="replace")


def check(status: int) -> None:
    if status != TG_OK:
        raise HipError(status, last_error() or load().tg_status_string(status).decode())


def device_count() -> int:
    n = ctypes.c_int(0)
    check(load().tg_device_count(ctypes.byref(n)))
    return int(n.value)
