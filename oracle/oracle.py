"""ctypes front end of the CPU oracle (``oracle/tg_oracle.c``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, always as the checker or the timed
CPU baseline, never as the thing measured or shipped.

Semantics restated (reference paths relative to the reference root):
``crates/tropical-gemm/src/types/scalar.rs:32-126`` (identities, wrapping
integer ops), ``types/max_plus.rs:66-73`` / ``min_plus.rs:66-73`` /
``max_mul.rs:65-72`` (first-k select rule), ``core/gemm.rs:167-244`` and
``core/kernel.rs:119-167`` (ascending global k), ``api.rs:563-646`` (backward
loop order) and ``crates/tropical-gemm-python/src/lib.rs:877-950`` (MaxMul
backward).  Everything is row-major.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libtg_oracle.so")

SEMIRINGS = {"maxplus": 0, "minplus": 1, "maxmul": 2}
_DT = {
    np.dtype(np.float32): ("f32", ctypes.c_float),
    np.dtype(np.float64): ("f64", ctypes.c_double),
    np.dtype(np.int32): ("i32", ctypes.c_int32),
    np.dtype(np.int64): ("i64", ctypes.c_int64),
}

_lib = None


def build() -> str:
    """Compile ``libtg_oracle.so`` in place (gcc, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        vp = ctypes.c_void_p
        i64 = ctypes.c_int64
        for name in ("f32", "f64", "i32", "i64"):
            fn = getattr(lib, f"tgo_gemm_{name}")
            fn.argtypes = [ctypes.c_int, vp, vp, vp, vp, i64, i64, i64, ctypes.c_int]
            fn.restype = ctypes.c_int
        for name in ("tgo_backward_a_f32", "tgo_backward_a_f64", "tgo_backward_b_f32",
                     "tgo_backward_b_f64"):
            fn = getattr(lib, name)
            fn.argtypes = [vp, vp, vp, vp, i64, i64, i64]
            fn.restype = None
        for name in ("tgo_portable_argmax_f32", "tgo_portable_argmax_f64", "tgo_portable_argmax_i32",
                     "tgo_portable_argmax_i64"):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.c_int, vp, vp, vp, vp, i64, i64, i64]
            fn.restype = ctypes.c_int
        for name in ("tgo_portable_gemm_i32", "tgo_portable_gemm_i64"):
            fn = getattr(lib, name)
            fn.argtypes = [ctypes.c_int, vp, vp, vp, i64, i64, i64]
            fn.restype = ctypes.c_int
        lib.tgo_avx2_gemm_f32.argtypes = [ctypes.c_int, vp, vp, vp, i64, i64, i64]
        lib.tgo_avx2_gemm_f32.restype = ctypes.c_int
        lib.tgo_avx2_gemm_maxplus_f64.argtypes = [vp, vp, vp, i64, i64, i64]
        lib.tgo_avx2_gemm_maxplus_f64.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _threads(n: int | None) -> int:
    if n is not None:
        return max(1, int(n))
    return max(1, min(16, os.cpu_count() or 1))


def gemm(semiring: str, a: np.ndarray, b: np.ndarray, with_argmax: bool = True,
         nthreads: int | None = None):
    """Row-major ``C = A (x) B``.  Returns ``(C, argmax)`` (argmax is uint32,
    ``None`` when ``with_argmax`` is False)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[0]:
        raise ValueError(f"shape mismatch: {a.shape} x {b.shape}")
    if a.dtype != b.dtype or a.dtype not in _DT:
        raise TypeError(f"unsupported dtypes {a.dtype}, {b.dtype}")
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=a.dtype)
    am = np.empty((m, n), dtype=np.uint32) if with_argmax else None
    name = _DT[a.dtype][0]
    rc = getattr(_load(), f"tgo_gemm_{name}")(SEMIRINGS[semiring], _ptr(a), _ptr(b), _ptr(c),
                                            _ptr(am), m, n, k, _threads(nthreads))
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return c, am


def gemm_batched(semiring: str, a: np.ndarray, b: np.ndarray, with_argmax: bool = True,
                 nthreads: int | None = None):
    """Batched row-major product: ``C[t] = A[t] (x) B[t]``."""
    cs, ams = [], []
    for t in range(a.shape[0]):
        c, am = gemm(semiring, a[t], b[t], with_argmax, nthreads)
        cs.append(c)
        ams.append(am)
    return np.stack(cs), (np.stack(ams) if with_argmax else None)


def backward_a(grad_c: np.ndarray, argmax: np.ndarray, k: int, b: np.ndarray | None = None):
    """``grad_a[i, argmax[i,j]] += grad_c[i,j]`` (times ``B[argmax,j]`` for MaxMul),
    visiting i then j ascending (api.rs:563-582, python/src/lib.rs:877-904)."""
    grad_c = np.ascontiguousarray(grad_c)
    am = np.ascontiguousarray(argmax).astype(np.uint32, copy=False)
    m, n = grad_c.shape
    out = np.empty((m, k), dtype=grad_c.dtype)
    name = {np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}[grad_c.dtype]
    bb = None if b is None else np.ascontiguousarray(b, dtype=grad_c.dtype)
    getattr(_load(), f"tgo_backward_a_{name}")(_ptr(grad_c), _ptr(am), _ptr(bb), _ptr(out), m, n, k)
    return out


def backward_b(grad_c: np.ndarray, argmax: np.ndarray, k: int, a: np.ndarray | None = None):
    """``grad_b[argmax[i,j], j] += grad_c[i,j]`` (times ``A[i,argmax]`` for MaxMul),
    visiting i then j ascending (api.rs:627-646, python/src/lib.rs:912-950)."""
    grad_c = np.ascontiguousarray(grad_c)
    am = np.ascontiguousarray(argmax).astype(np.uint32, copy=False)
    m, n = grad_c.shape
    out = np.empty((k, n), dtype=grad_c.dtype)
    name = {np.dtype(np.float32): "f32", np.dtype(np.float64): "f64"}[grad_c.dtype]
    aa = None if a is None else np.ascontiguousarray(a, dtype=grad_c.dtype)
    getattr(_load(), f"tgo_backward_b_{name}")(_ptr(grad_c), _ptr(am), _ptr(aa), _ptr(out), m, n, k)
    return out


def portable_argmax(semiring: str, a: np.ndarray, b: np.ndarray):
    """Single-thread restatement of the reference CPU argmax path (BLIS
    PORTABLE tiling + 4x4 scalar microkernel) for float32, float64, int32 or
    int64 operands; used as the timed baseline."""
    dt = np.dtype(a.dtype)
    if dt not in (np.dtype(np.float32), np.dtype(np.float64), np.dtype(np.int32),
                  np.dtype(np.int64)):
        raise ValueError(f"portable baseline restated for float32, float64, int32 and int64, got {dt}")
    a = np.ascontiguousarray(a, dtype=dt)
    b = np.ascontiguousarray(b, dtype=dt)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=dt)
    am = np.empty((m, n), dtype=np.uint32)
    fn = {np.dtype(np.float32): _load().tgo_portable_argmax_f32,
          np.dtype(np.float64): _load().tgo_portable_argmax_f64,
          np.dtype(np.int32): _load().tgo_portable_argmax_i32,
          np.dtype(np.int64): _load().tgo_portable_argmax_i64}[dt]
    rc = fn(SEMIRINGS[semiring], _ptr(a), _ptr(b), _ptr(c), _ptr(am), m, n, k)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return c, am


def portable_argmax_f32(semiring: str, a: np.ndarray, b: np.ndarray):
    """float32 form of ``portable_argmax``."""
    return portable_argmax(semiring, np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32))


def portable_gemm(semiring: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Single-thread restatement of the reference CPU value-only path for
    integer operands (BLIS PORTABLE tiling + 4x4 value microkernel,
    core/kernel.rs:72-117; simd/dispatch.rs:233-242 sends every i32 / i64
    semiring there); used as the timed baseline of value-only integer
    configurations."""
    dt = np.dtype(a.dtype)
    if dt not in (np.dtype(np.int32), np.dtype(np.int64)):
        raise ValueError(f"portable value baseline restated for int32 and int64, got {dt}")
    a = np.ascontiguousarray(a, dtype=dt)
    b = np.ascontiguousarray(b, dtype=dt)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=dt)
    fn = {np.dtype(np.int32): _load().tgo_portable_gemm_i32,
          np.dtype(np.int64): _load().tgo_portable_gemm_i64}[dt]
    rc = fn(SEMIRINGS[semiring], _ptr(a), _ptr(b), _ptr(c), m, n, k)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return c


def avx2_gemm_maxplus_f64(semiring: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Single-thread restatement of the reference CPU value-only MaxPlus f64
    path (BLIS F64_AVX2 tiling + AVX2 4x4 f64 microkernel,
    simd/kernels/avx2.rs:77-143); used as the timed baseline of value-only
    f64 MaxPlus configurations.  The reference runs MinPlus and MaxMul f64
    on its portable path, which has no value-only restatement here."""
    if semiring != "maxplus":
        raise ValueError("the reference's AVX2 f64 kernel is MaxPlus only")
    a = np.ascontiguousarray(a, dtype=np.float64)
    b = np.ascontiguousarray(b, dtype=np.float64)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=np.float64)
    rc = _load().tgo_avx2_gemm_maxplus_f64(_ptr(a), _ptr(b), _ptr(c), m, n, k)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return c


def avx2_gemm_f32(semiring: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Single-thread restatement of the reference CPU value-only f32 path
    (BLIS F32_AVX2 tiling + AVX2 8x8 microkernel); used as the timed
    baseline of value-only configurations."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=np.float32)
    rc = _load().tgo_avx2_gemm_f32(SEMIRINGS[semiring], _ptr(a), _ptr(b), _ptr(c), m, n, k)
    if rc != 0:
        raise ValueError("oracle rejected arguments")
    return c
