"""PyTorch autograd functions for tropical matmul on MI355X.

Mirrors the GPU and batched classes of the reference
(``crates/tropical-gemm-python/python/tropical_gemm/pytorch.py:338-860``):
same class and function names, same forward outputs, same gradient rules.

Differences that are deliberate:

* The backward runs the library's HIP scatter kernels (``tg_backward_*``)
  instead of ``torch.scatter_add_`` (reference ``pytorch.py:386-403``);
  the math is identical: ``grad_a[i, k*] += grad_c[i, j]``,
  ``grad_b[k*, j] += grad_c[i, j]`` and, for MaxMul, the multiplicative rule
  ``grad_a[i, k*] += grad_c[i, j] * B[k*, j]``, ``grad_b[k*, j] += grad_c[i, j] * A[i, k*]``
  (``pytorch.py:521-548``).
* float32 and float64 are both accepted on the GPU (the reference's DLPack
  path takes float32 only, ``python/src/lib.rs:2193-2197``).
* The argmax saved for backward stays int32 on the device (the reference
  widens it to int64 for ``scatter_add_``).
* The reference's CPU autograd classes (Rust SIMD backend) are not part of
  this backend; the batched classes require device tensors.
"""
from __future__ import annotations

import torch

from . import cuda_available, ops

GPU_AVAILABLE = cuda_available()
_DLPACK_AVAILABLE = True
_BATCHED_DLPACK_AVAILABLE = True

_GRAD_DTYPES = (torch.float32, torch.float64)


def _prep(a: torch.Tensor, b: torch.Tensor, name: str, cpu_name: str):
    if not a.is_cuda:
        raise RuntimeError(f"{name} requires GPU tensors. Use {cpu_name} for CPU tensors.")
    if a.device != b.device:
        raise RuntimeError(
            f"Tensors must be on the same device: a is on {a.device}, b is on {b.device}")
    if a.dtype not in _GRAD_DTYPES or b.dtype != a.dtype:
        raise RuntimeError(f"{name} supports float32/float64 tensors of one dtype, got "
                           f"{a.dtype} and {b.dtype}")
    return a.detach().contiguous(), b.detach().contiguous()


def _additive_forward(ctx, a, b, semiring: str, name: str, cpu_name: str):
    a_c, b_c = _prep(a, b, name, cpu_name)
    c, argmax = ops.gemm(semiring, a_c, b_c, True)
    ctx.save_for_backward(argmax)
    ctx.k = a.shape[1]
    ctx.m = a.shape[0]
    ctx.n = b.shape[1]
    return c


class _AdditiveGPU(torch.autograd.Function):

    @staticmethod
    def backward(ctx, grad_c: torch.Tensor):
        (argmax,) = ctx.saved_tensors
        grad_a = grad_b = None
        if ctx.needs_input_grad[0]:
            grad_a = ops.backward_a(grad_c, argmax, ctx.k)
        if ctx.needs_input_grad[1]:
            grad_b = ops.backward_b(grad_c, argmax, ctx.k)
        return grad_a, grad_b


class TropicalMaxPlusMatmulGPU(_AdditiveGPU):
    """GPU MaxPlus matmul ``C[i,j] = max_k A[i,k] + B[k,j]`` (pytorch.py:338-403)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        return _additive_forward(ctx, a, b, "maxplus", "TropicalMaxPlusMatmulGPU",
                                 "TropicalMaxPlusMatmul")


class TropicalMinPlusMatmulGPU(_AdditiveGPU):
    """GPU MinPlus matmul ``C[i,j] = min_k A[i,k] + B[k,j]`` (pytorch.py:406-468)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        return _additive_forward(ctx, a, b, "minplus", "TropicalMinPlusMatmulGPU",
                                 "TropicalMinPlusMatmul")


class TropicalMaxMulMatmulGPU(torch.autograd.Function):
    """GPU MaxMul matmul ``C[i,j] = max_k A[i,k] * B[k,j]`` with the
    multiplicative backward (pytorch.py:471-548)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        a_c, b_c = _prep(a, b, "TropicalMaxMulMatmulGPU", "TropicalMaxMulMatmul")
        c, argmax = ops.gemm("maxmul", a_c, b_c, True)
        ctx.save_for_backward(a_c, b_c, argmax)
        ctx.k = a.shape[1]
        ctx.m = a.shape[0]
        ctx.n = b.shape[1]
        return c

    @staticmethod
    def backward(ctx, grad_c: torch.Tensor):
        a, b, argmax = ctx.saved_tensors
        grad_a = grad_b = None
        if ctx.needs_input_grad[0]:
            grad_a = ops.backward_a(grad_c, argmax, ctx.k, b=b)
        if ctx.needs_input_grad[1]:
            grad_b = ops.backward_b(grad_c, argmax, ctx.k, a=a)
        return grad_a, grad_b


def _prep_batched(a: torch.Tensor, b: torch.Tensor):
    if not (a.is_cuda or b.is_cuda):
        raise RuntimeError("Batched tropical matmul on this backend requires GPU tensors; the "
                           "reference's CPU batched path is not part of it.")
    if a.device != b.device:
        raise RuntimeError(
            f"Tensors must be on the same device: a is on {a.device}, b is on {b.device}")
    if a.dtype not in _GRAD_DTYPES or b.dtype != a.dtype:
        raise RuntimeError(f"Batched GPU tropical matmul supports float32/float64 tensors of one "
                           f"dtype, got {a.dtype} and {b.dtype}")
    return a.detach().contiguous(), b.detach().contiguous()


def _additive_batched_forward(ctx, a, b, semiring: str):
    a_c, b_c = _prep_batched(a, b)
    c, argmax = ops.gemm_batched(semiring, a_c, b_c, True)
    ctx.save_for_backward(argmax)
    ctx.k = a.shape[2]
    ctx.batch = a.shape[0]
    ctx.m = a.shape[1]
    ctx.n = b.shape[2]
    return c


class _AdditiveBatched(torch.autograd.Function):

    @staticmethod
    def backward(ctx, grad_c: torch.Tensor):
        (argmax,) = ctx.saved_tensors
        grad_a = grad_b = None
        if ctx.needs_input_grad[0]:
            grad_a = ops.backward_a_batched(grad_c, argmax, ctx.k)
        if ctx.needs_input_grad[1]:
            grad_b = ops.backward_b_batched(grad_c, argmax, ctx.k)
        return grad_a, grad_b


class TropicalMaxPlusMatmulBatched(_AdditiveBatched):
    """Batched MaxPlus ``C[b,i,j] = max_k A[b,i,k] + B[b,k,j]`` (pytorch.py:556-640)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        return _additive_batched_forward(ctx, a, b, "maxplus")


class TropicalMinPlusMatmulBatched(_AdditiveBatched):
    """Batched MinPlus ``C[b,i,j] = min_k A[b,i,k] + B[b,k,j]`` (pytorch.py:643-730)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        return _additive_batched_forward(ctx, a, b, "minplus")


class TropicalMaxMulMatmulBatched(torch.autograd.Function):
    """Batched MaxMul with the multiplicative backward (pytorch.py:733-832)."""

    @staticmethod
    def forward(ctx, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        a_c, b_c = _prep_batched(a, b)
        c, argmax = ops.gemm_batched("maxmul", a_c, b_c, True)
        ctx.save_for_backward(a_c, b_c, argmax)
        ctx.k = a.shape[2]
        ctx.batch = a.shape[0]
        ctx.m = a.shape[1]
        ctx.n = b.shape[2]
        return c

    @staticmethod
    def backward(ctx, grad_c: torch.Tensor):
        a, b, argmax = ctx.saved_tensors
        grad_a = grad_b = None
        if ctx.needs_input_grad[0]:
            grad_a = ops.backward_a_batched(grad_c, argmax, ctx.k, b=b)
        if ctx.needs_input_grad[1]:
            grad_b = ops.backward_b_batched(grad_c, argmax, ctx.k, a=a)
        return grad_a, grad_b


def tropical_maxplus_matmul_gpu(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """GPU MaxPlus tropical matmul (pytorch.py:910-924)."""
    return TropicalMaxPlusMatmulGPU.apply(a, b)


def tropical_minplus_matmul_gpu(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """GPU MinPlus tropical matmul (pytorch.py:927-941)."""
    return TropicalMinPlusMatmulGPU.apply(a, b)


def tropical_maxmul_matmul_gpu(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """GPU MaxMul tropical matmul (pytorch.py:944-958)."""
    return TropicalMaxMulMatmulGPU.apply(a, b)


def tropical_maxplus_matmul_batched(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Batched MaxPlus tropical matmul (pytorch.py:961-973)."""
    return TropicalMaxPlusMatmulBatched.apply(a, b)


def tropical_minplus_matmul_batched(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Batched MinPlus tropical matmul (pytorch.py:976-988)."""
    return TropicalMinPlusMatmulBatched.apply(a, b)


def tropical_maxmul_matmul_batched(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Batched MaxMul tropical matmul (pytorch.py:991-1003)."""
    return TropicalMaxMulMatmulBatched.apply(a, b)


__all__ = [
    "TropicalMaxPlusMatmulGPU",
    "TropicalMinPlusMatmulGPU",
    "TropicalMaxMulMatmulGPU",
    "TropicalMaxPlusMatmulBatched",
    "TropicalMinPlusMatmulBatched",
    "TropicalMaxMulMatmulBatched",
    "tropical_maxplus_matmul_gpu",
    "tropical_minplus_matmul_gpu",
    "tropical_maxmul_matmul_gpu",
    "tropical_maxplus_matmul_batched",
    "tropical_minplus_matmul_batched",
    "tropical_maxmul_matmul_batched",
    "GPU_AVAILABLE",
    "_DLPACK_AVAILABLE",
]
