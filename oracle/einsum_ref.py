"""Brute-force CPU restatement of tropical einsum -- test infrastructure only.

Only ``tests/`` may import this module; the product path never does.

The reference does not implement tropical einsum: it is a design plan
(``docs/plans/2026-01-26-tropical-einsum-design.md:245-300`` for the binary
contraction, ``:340-430`` for the engine).  This restatement follows the
definition instead, by enumerating index assignments (pure Python loops,
small tensors only):

* ``contract_binary_ref``: ``Y[y] = (+)_{assignments of the non-output
  labels} A[..] (x) B[..]``, visiting the contracted labels (in their order
  of appearance in ``ia``) in row-major order and keeping the first strict
  improvement, as the reference's CPU GEMM does for its k loop
  (``crates/tropical-gemm/src/types/max_plus.rs:66-73``).  Labels that
  appear in one operand only are enumerated together with the contracted
  ones; the argmax is defined only when there are none.
* ``einsum_ref``: the same enumeration over every operand, multiplying the
  operands left to right.  With more than two operands float results depend
  on the association, so tests use integer-exact data for those.

Pinned by ``tests/test_einsum_cpu.py``: a plain matrix product equals
``oracle.gemm`` (itself pinned by the reference's golden fixtures), and the
closed forms of a dot product, an outer product, a trace and a full
reduction.
"""
from __future__ import annotations

import itertools

import numpy as np

_JOIN = {"maxplus": max, "minplus": min, "maxmul": max}


def _zero(semiring, dtype):
    dtype = np.dtype(dtype)
    if dtype.kind == "f":
        return {"maxplus": -np.inf, "minplus": np.inf, "maxmul": 0.0}[semiring]
    info = np.iinfo(dtype)
    return {"maxplus": int(info.min), "minplus": int(info.max), "maxmul": 0}[semiring]


def _mul(semiring, x, y, dtype):
    dtype = np.dtype(dtype)
    if dtype.kind == "f":
        x, y = dtype.type(x), dtype.type(y)
        return x * y if semiring == "maxmul" else x + y
    bits = dtype.itemsize * 8
    v = (int(x) * int(y)) if semiring == "maxmul" else (int(x) + int(y))
    v &= (1 << bits) - 1  # two's-complement wraparound
    return v - (1 << bits) if v >> (bits - 1) else v


def _better(semiring, cand, acc):
    return cand < acc if semiring == "minplus" else cand > acc


def contract_binary_ref(a, b, ia, ib, iy, semiring="maxplus"):
    """Returns ``(Y, argmax)``; ``argmax`` is None when a label is summed in
    one operand only."""
    a = np.asarray(a)
    b = np.asarray(b)
    ia, ib, iy = list(ia), list(ib), list(iy)
    size = {x: a.shape[p] for p, x in enumerate(ia)}
    size.update({x: b.shape[p] for p, x in enumerate(ib)})
    con = [x for x in ia if x in ib and x not in iy]
    one_side = [x for x in ia + ib if x not in iy and x not in con]
    summed = con + [x for x in one_side if x not in con]
    summed = list(dict.fromkeys(summed))
    dtype = a.dtype
    y = np.empty([size[x] for x in iy], dtype=dtype)
    idx = np.zeros([size[x] for x in iy], dtype=np.int64)
    for out in itertools.product(*[range(size[x]) for x in iy]):
        env = dict(zip(iy, out))
        acc = _zero(semiring, dtype)
        best = 0
        for pos, s in enumerate(itertools.product(*[range(size[x]) for x in summed])):
            env.update(zip(summed, s))
            p = _mul(semiring, a[tuple(env[x] for x in ia)], b[tuple(env[x] for x in ib)], dtype)
            if _better(semiring, p, acc):
                acc = p
                best = pos
        y[out] = acc
        idx[out] = best
    return y, (None if one_side else idx)


def einsum_ref(ixs, iy, operands, semiring="maxplus"):
    """Tropical einsum by enumeration; operands multiplied left to right."""
    ops_ = [np.asarray(t) for t in operands]
    size = {}
    for t, lab in zip(ops_, ixs):
        for p, x in enumerate(lab):
            size[x] = t.shape[p]
    summed = list(dict.fromkeys(x for lab in ixs for x in lab if x not in iy))
    dtype = ops_[0].dtype
    y = np.empty([size[x] for x in iy], dtype=dtype)
    for out in itertools.product(*[range(size[x]) for x in iy]):
        env = dict(zip(iy, out))
        acc = _zero(semiring, dtype)
        for s in itertools.product(*[range(size[x]) for x in summed]):
            env.update(zip(summed, s))
            p = None
            for t, lab in zip(ops_, ixs):
                v = t[tuple(env[x] for x in lab)]
                p = v if p is None else _mul(semiring, p, v, dtype)
            if _better(semiring, p, acc):
                acc = p
        y[out] = acc
    return y
