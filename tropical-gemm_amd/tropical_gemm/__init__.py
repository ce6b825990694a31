"""tropical_gemm -- MI355X (gfx950) backend of tropical matrix multiplication.

Python face of the HIP library, mirroring the GPU half of the reference
package ``tropical_gemm`` (``crates/tropical-gemm-python/python/tropical_gemm/__init__.py``
and the ``mod gpu`` functions of ``crates/tropical-gemm-python/src/lib.rs:1657-2601``):

* numpy in / numpy out: ``{maxplus,minplus,maxmul}_matmul_gpu`` and
  ``..._gpu_with_argmax`` (lib.rs:1885-2080; here row-major-correct for every
  shape, see the note below);
* zero-copy device tensors: ``{maxplus,minplus,maxmul}_matmul_dlpack`` and
  ``..._batched_dlpack`` returning DLPack capsules (lib.rs:2105-2563);
* ``cuda_available()`` (lib.rs:2341-2344), true when a HIP device and the
  native library are present.

The reference's numpy GPU functions hand row-major numpy data to its
column-major API without the operand swap (lib.rs:1904-1907), which is wrong
for non-symmetric inputs; these functions compute the row-major product.

Argmax arrays are int32 (the reference GPU's ``ArgmaxIndex``), values of the
first k attaining each output.  The CPU (numpy, Rust SIMD) half of the
reference package is not part of this backend.
"""
from __future__ import annotations

import numpy as np

from . import _native
from ._native import HipError

__version__ = "0.1.0"

_NP_DT = {np.dtype(np.float32): "f32", np.dtype(np.float64): "f64",
          np.dtype(np.int32): "i32", np.dtype(np.int64): "i64"}


def cuda_available() -> bool:
    """True when the native library loads and at least one HIP device exists."""
    try:
        return _native.device_count() > 0
    except Exception:
        return False


def _torch():
    import torch  # local: torch is only needed for the device entry points

    return torch


def _numpy_gpu(semiring: str, a, b, with_argmax: bool):
    torch = _torch()
    from . import ops

    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError(f"Expected 2D arrays, got A with {a.ndim} dims, B with {b.ndim} dims")
    m, k = a.shape
    if k != b.shape[0]:
        raise ValueError(f"Dimension mismatch: A is {m}x{k}, B is {b.shape[0]}x{b.shape[1]}")
    if a.dtype != b.dtype or a.dtype not in _NP_DT:
        raise ValueError(f"unsupported dtypes {a.dtype}/{b.dtype}")
    dev = torch.device("cuda", 0)
    ta = torch.from_numpy(a).to(dev)
    tb = torch.from_numpy(b).to(dev)
    c, am = ops.gemm(semiring, ta, tb, with_argmax)
    torch.cuda.synchronize(dev)  # blocking, like the reference (kernels.rs:65)
    c_np = c.cpu().numpy().reshape(-1)
    if with_argmax:
        return c_np, am.cpu().numpy().reshape(-1)
    return c_np


def maxplus_matmul_gpu(a, b):
    """MaxPlus ``C[i,j] = max_k A[i,k] + B[k,j]`` on the GPU; flattened result."""
    return _numpy_gpu("maxplus", a, b, False)


def minplus_matmul_gpu(a, b):
    """MinPlus ``C[i,j] = min_k A[i,k] + B[k,j]`` on the GPU; flattened result."""
    return _numpy_gpu("minplus", a, b, False)


def maxmul_matmul_gpu(a, b):
    """MaxMul ``C[i,j] = max_k A[i,k] * B[k,j]`` on the GPU; flattened result."""
    return _numpy_gpu("maxmul", a, b, False)


def maxplus_matmul_gpu_with_argmax(a, b):
    """MaxPlus with argmax; returns flattened ``(C, argmax)``."""
    return _numpy_gpu("maxplus", a, b, True)


def minplus_matmul_gpu_with_argmax(a, b):
    """MinPlus with argmin; returns flattened ``(C, argmax)``."""
    return _numpy_gpu("minplus", a, b, True)


def maxmul_matmul_gpu_with_argmax(a, b):
    """MaxMul with argmax; returns flattened ``(C, argmax)``."""
    return _numpy_gpu("maxmul", a, b, True)


def _dlpack_2d(semiring: str, a, b):
    torch = _torch()
    from . import ops

    a = ops.as_tensor(a)
    b = ops.as_tensor(b)
    if a.dim() == 2 and b.dim() == 2 and (0 in a.shape or 0 in b.shape):
        raise ValueError(f"Zero-sized dimensions not supported: m={a.shape[0]}, k={a.shape[1]}, "
                         f"n={b.shape[1]}")
    c, am = ops.gemm(semiring, a, b, True)
    return torch.utils.dlpack.to_dlpack(c), torch.utils.dlpack.to_dlpack(am)


def _dlpack_3d(semiring: str, a, b):
    torch = _torch()
    from . import ops

    a = ops.as_tensor(a)
    b = ops.as_tensor(b)
    if a.device.type != "cuda":
        raise RuntimeError(f"Tensor A must be on a GPU device, got {a.device.type}.")
    if b.device.type != "cuda":
        raise RuntimeError(f"Tensor B must be on a GPU device, got {b.device.type}.")
    if a.dim() == 3 and b.dim() == 3 and (0 in a.shape or 0 in b.shape):
        raise ValueError(f"Zero-sized dimensions not supported: batch={a.shape[0]}, m={a.shape[1]}, "
                         f"k={a.shape[2]}, n={b.shape[2]}")
    c, am = ops.gemm_batched(semiring, a, b, True)
    return torch.utils.dlpack.to_dlpack(c), torch.utils.dlpack.to_dlpack(am)


def maxplus_matmul_dlpack(a, b):
    """MaxPlus + argmax on device tensors; returns DLPack capsules ``(C, argmax)``."""
    return _dlpack_2d("maxplus", a, b)


def minplus_matmul_dlpack(a, b):
    """MinPlus + argmin on device tensors; returns DLPack capsules ``(C, argmax)``."""
    return _dlpack_2d("minplus", a, b)


def maxmul_matmul_dlpack(a, b):
    """MaxMul + argmax on device tensors; returns DLPack capsules ``(C, argmax)``."""
    return _dlpack_2d("maxmul", a, b)


def maxplus_matmul_batched_dlpack(a, b):
    """Batched MaxPlus + argmax on 3-D device tensors; DLPack capsules."""
    return _dlpack_3d("maxplus", a, b)


def minplus_matmul_batched_dlpack(a, b):
    """Batched MinPlus + argmin on 3-D device tensors; DLPack capsules."""
    return _dlpack_3d("minplus", a, b)


def maxmul_matmul_batched_dlpack(a, b):
    """Batched MaxMul + argmax on 3-D device tensors; DLPack capsules."""
    return _dlpack_3d("maxmul", a, b)


__all__ = [
    "HipError",
    "cuda_available",
    "maxplus_matmul_gpu",
    "minplus_matmul_gpu",
    "maxmul_matmul_gpu",
    "maxplus_matmul_gpu_with_argmax",
    "minplus_matmul_gpu_with_argmax",
    "maxmul_matmul_gpu_with_argmax",
    "maxplus_matmul_dlpack",
    "minplus_matmul_dlpack",
    "maxmul_matmul_dlpack",
    "maxplus_matmul_batched_dlpack",
    "minplus_matmul_batched_dlpack",
    "maxmul_matmul_batched_dlpack",
]
