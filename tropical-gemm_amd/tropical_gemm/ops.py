"""Tensor-level entry points over the C ABI (device tensors in, device tensors out).

These are the operations the reference reaches through its DLPack path:
``dlpack_2d_impl`` / ``batched_dlpack_impl``
(``crates/tropical-gemm-python/src/lib.rs:2149-2338``, ``:2418-2563``) for the
forward, and the GPU backward kernels (``crates/tropical-gemm-cuda/src/lib.rs:841-942``)
for the scatter.  Inputs are PyTorch-ROCm tensors (any DLPack producer is
accepted by ``as_tensor``); outputs are allocated with torch's caching
allocator on the input's device, and every launch goes to torch's current
stream of that device, so results are ordered with surrounding torch work.
Workspaces also come from torch's allocator (no hipMalloc on the hot path).
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as nat

_DT = {torch.float32: "f32", torch.float64: "f64", torch.int32: "i32", torch.int64: "i64"}
_FLOAT = (torch.float32, torch.float64)


def as_tensor(x) -> torch.Tensor:
    """Accept a torch tensor or any object implementing ``__dlpack__``."""
    if isinstance(x, torch.Tensor):
        return x
    if hasattr(x, "__dlpack__"):
        return torch.utils.dlpack.from_dlpack(x)
    raise TypeError(f"expected a tensor or a DLPack producer, got {type(x).__name__}")


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check_pair(a: torch.Tensor, b: torch.Tensor, ndim: int) -> None:
    # Same checks, same order, as dlpack_2d_impl (python/src/lib.rs:2165-2245).
    if a.device.type != b.device.type:
        raise ValueError(f"Tensors must be on the same device type: A is on {a.device.type}, "
                         f"B is on {b.device.type}")
    if a.device != b.device:
        raise ValueError(f"Tensors must be on the same device: A is on {a.device}, B is on {b.device}")
    if a.dtype != b.dtype:
        raise ValueError(f"Tensors must have the same dtype: A is {a.dtype}, B is {b.dtype}")
    if a.dtype not in _DT:
        raise ValueError(f"Unsupported dtype {a.dtype}: expected float32, float64, int32 or int64")
    if a.dim() != ndim or b.dim() != ndim:
        raise ValueError(f"Expected {ndim}D tensors, got A with {a.dim()} dims, B with {b.dim()} dims")
    if a.device.type != "cuda":
        raise ValueError("tropical_gemm GPU entry points need device tensors "
                         f"(got {a.device.type}); move the tensors to the GPU first")


def gemm(semiring: str, a, b, with_argmax: bool = True):
    """Row-major ``C = A (x) B`` on the GPU.  Returns ``(C, argmax)`` with
    ``argmax`` int32 (``None`` when ``with_argmax`` is False)."""
    a = as_tensor(a)
    b = as_tensor(b)
    _check_pair(a, b, 2)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"Dimension mismatch: A is {m}x{k}, B is {k2}x{n}")
    if not a.is_contiguous() or not b.is_contiguous():
        raise ValueError("Tensors must be contiguous (call .contiguous() on PyTorch tensors)")
    dev = a.device
    c = torch.empty((m, n), dtype=a.dtype, device=dev)
    am = torch.empty((m, n), dtype=torch.int32, device=dev) if with_argmax else None
    lib = nat.load()
    dt = nat.DTYPE[_DT[a.dtype]]
    ws_bytes = lib.tg_gemm_workspace_size(dt, 1, m, n, k, 1 if with_argmax else 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    nat.check(lib.tg_gemm_ws(dev.index or 0, nat.SEMIRING[semiring], dt, nat.LAYOUT["row"],
                             _ptr(a), _ptr(b), _ptr(c), _ptr(am), m, n, k, _ptr(ws), ws_bytes,
                             _stream(dev)))
    return c, am


def gemm_batched(semiring: str, a, b, with_argmax: bool = True):
    """Batched row-major product ``C[t] = A[t] (x) B[t]`` for 3-D tensors."""
    a = as_tensor(a)
    b = as_tensor(b)
    _check_pair(a, b, 3)
    batch, m, k = a.shape
    batch_b, k2, n = b.shape
    if batch != batch_b:
        raise ValueError(f"Batch size mismatch: A has batch {batch}, B has batch {batch_b}")
    if k != k2:
        raise ValueError(f"Dimension mismatch: A is (batch, {m}, {k}), B is (batch, {k2}, {n})")
    if not a.is_contiguous() or not b.is_contiguous():
        raise ValueError("Tensors must be contiguous (call .contiguous() on PyTorch tensors)")
    dev = a.device
    c = torch.empty((batch, m, n), dtype=a.dtype, device=dev)
    am = torch.empty((batch, m, n), dtype=torch.int32, device=dev) if with_argmax else None
    lib = nat.load()
    dt = nat.DTYPE[_DT[a.dtype]]
    ws_bytes = lib.tg_gemm_workspace_size(dt, batch, m, n, k, 1 if with_argmax else 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    nat.check(lib.tg_gemm_strided_batched_ws(
        dev.index or 0, nat.SEMIRING[semiring], dt, nat.LAYOUT["row"], _ptr(a), _ptr(b), _ptr(c),
        _ptr(am), batch, m, n, k, m * k, k * n, m * n, _ptr(ws), ws_bytes, _stream(dev)))
    return c, am


def _check_backward(grad_c: torch.Tensor, argmax: torch.Tensor, ndim: int):
    if grad_c.dtype not in _FLOAT:
        raise ValueError(f"gradients are defined for float32/float64, got {grad_c.dtype}")
    if argmax.dtype != torch.int32:
        raise ValueError(f"argmax must be int32, got {argmax.dtype}")
    if grad_c.shape != argmax.shape or grad_c.dim() != ndim:
        raise ValueError(f"grad_c {tuple(grad_c.shape)} and argmax {tuple(argmax.shape)} must "
                         f"have the same {ndim}-D shape")
    if grad_c.device != argmax.device or grad_c.device.type != "cuda":
        raise ValueError("grad_c and argmax must be on the same GPU")


def backward_a(grad_c: torch.Tensor, argmax: torch.Tensor, k: int,
               b: torch.Tensor | None = None) -> torch.Tensor:
    """``grad_a[i, argmax[i,j]] += grad_c[i,j]`` (times ``B[argmax, j]`` when
    ``b`` is given: the MaxMul rule).  Returns a new (m, k) tensor."""
    grad_c = grad_c.contiguous()
    argmax = argmax.contiguous()
    _check_backward(grad_c, argmax, 2)
    m, n = grad_c.shape
    dev = grad_c.device
    out = torch.empty((m, k), dtype=grad_c.dtype, device=dev)
    lib = nat.load()
    dt = nat.DTYPE[_DT[grad_c.dtype]]
    if b is None:
        nat.check(lib.tg_backward_a(dev.index or 0, dt, 0, _ptr(grad_c), _ptr(argmax), _ptr(out),
                                    m, n, k, _stream(dev)))
    else:
        b = b.to(dtype=grad_c.dtype).contiguous()
        nat.check(lib.tg_maxmul_backward_a(dev.index or 0, dt, 0, _ptr(grad_c), _ptr(argmax),
                                           _ptr(b), _ptr(out), m, n, k, _stream(dev)))
    return out


def backward_b(grad_c: torch.Tensor, argmax: torch.Tensor, k: int,
               a: torch.Tensor | None = None) -> torch.Tensor:
    """``grad_b[argmax[i,j], j] += grad_c[i,j]`` (times ``A[i, argmax]`` when
    ``a`` is given: the MaxMul rule).  Returns a new (k, n) tensor."""
    grad_c = grad_c.contiguous()
    argmax = argmax.contiguous()
    _check_backward(grad_c, argmax, 2)
    m, n = grad_c.shape
    dev = grad_c.device
    out = torch.empty((k, n), dtype=grad_c.dtype, device=dev)
    lib = nat.load()
    dt = nat.DTYPE[_DT[grad_c.dtype]]
    if a is None:
        nat.check(lib.tg_backward_b(dev.index or 0, dt, 0, _ptr(grad_c), _ptr(argmax), _ptr(out),
                                    m, n, k, _stream(dev)))
    else:
        a = a.to(dtype=grad_c.dtype).contiguous()
        nat.check(lib.tg_maxmul_backward_b(dev.index or 0, dt, 0, _ptr(grad_c), _ptr(argmax),
                                           _ptr(a), _ptr(out), m, n, k, _stream(dev)))
    return out


def backward_a_batched(grad_c: torch.Tensor, argmax: torch.Tensor, k: int,
                       b: torch.Tensor | None = None) -> torch.Tensor:
    grad_c = grad_c.contiguous()
    argmax = argmax.contiguous()
    _check_backward(grad_c, argmax, 3)
    batch, m, n = grad_c.shape
    dev = grad_c.device
    out = torch.empty((batch, m, k), dtype=grad_c.dtype, device=dev)
    if b is not None:
        b = b.to(dtype=grad_c.dtype).contiguous()
    lib = nat.load()
    dt = nat.DTYPE[_DT[grad_c.dtype]]
    nat.check(lib.tg_backward_a_strided_batched(
        dev.index or 0, dt, 0, _ptr(grad_c), _ptr(argmax), _ptr(b), _ptr(out), batch, m, n, k,
        m * n, k * n, m * k, _stream(dev)))
    return out


def backward_b_batched(grad_c: torch.Tensor, argmax: torch.Tensor, k: int,
                       a: torch.Tensor | None = None) -> torch.Tensor:
    grad_c = grad_c.contiguous()
    argmax = argmax.contiguous()
    _check_backward(grad_c, argmax, 3)
    batch, m, n = grad_c.shape
    dev = grad_c.device
    out = torch.empty((batch, k, n), dtype=grad_c.dtype, device=dev)
    if a is not None:
        a = a.to(dtype=grad_c.dtype).contiguous()
    lib = nat.load()
    dt = nat.DTYPE[_DT[grad_c.dtype]]
    nat.check(lib.tg_backward_b_strided_batched(
        dev.index or 0, dt, 0, _ptr(grad_c), _ptr(argmax), _ptr(a), _ptr(out), batch, m, n, k,
        m * n, m * k, k * n, _stream(dev)))
    return out


def transpose(t: torch.Tensor) -> torch.Tensor:
    """``t.transpose(-1, -2).contiguous()`` of a contiguous 2-D or 3-D device
    tensor (3-D: a batch of matrices) through ``tg_transpose``; the data
    movement of the tropical einsum.  No autograd."""
    t = as_tensor(t)
    if t.dtype not in _DT:
        raise ValueError(f"Unsupported dtype {t.dtype}: expected float32, float64, int32 or int64")
    if t.device.type != "cuda":
        raise ValueError("tropical_gemm GPU entry points need device tensors")
    if t.dim() not in (2, 3) or not t.is_contiguous():
        raise ValueError("expected a contiguous 2-D or 3-D tensor")
    batch = t.shape[0] if t.dim() == 3 else 1
    rows, cols = t.shape[-2], t.shape[-1]
    out = torch.empty(t.shape[:-2] + (cols, rows), dtype=t.dtype, device=t.device)
    lib = nat.load()
    nat.check(lib.tg_transpose(t.device.index or 0, nat.DTYPE[_DT[t.dtype]], _ptr(t), _ptr(out),
                               batch, rows, cols, _stream(t.device)))
    return out
