"""Tropical einsum: tensor contractions executed as the library's GEMM.

The reference plans this caller in ``docs/plans/2026-01-26-tropical-einsum-design.md``
(not implemented there): a binary contraction classifies its indices into
batch / left / right / contracted, permutes and reshapes both operands into
one (batched) matrix product and reshapes the result back (:245-300); an
einsum engine runs a pairwise contraction tree (:340-430), ordered greedily
(``GreedyMethod::new(0.0, 0.0)``: the next pair is the one whose result is
smallest, :370-375).  This module is that caller over device tensors:

* ``contract_binary(a, b, ia, ib, iy, semiring, with_argmax)`` -- one
  contraction through ``tg_gemm_ws`` / ``tg_gemm_strided_batched_ws``;
* ``einsum(code, *operands, semiring, optimize)`` -- ``"ij,jk->ik"``-style
  codes over any number of operands, with repeated labels (diagonals),
  labels summed inside one operand, outer products and full reductions;
* ``einsum_path(ixs, iy, sizes, optimize)`` -- the contraction order alone.

Semantics.  With labels L and the semiring's (+) (max or min) and (x) (+ or
*), ``Y[y] = (+) over every assignment of the labels not in the output of
(x) over the operands``.  A binary contraction computes one (x) per term and
keeps the first strict improvement in the row-major order of the contracted
labels (the GEMM's k order), so its values are those of the definition bit
for bit; a longer chain associates as the contraction tree does.  Labels
summed inside one operand are reduced first, as a product with a column of
the semiring's one (0 for MaxPlus/MinPlus, 1 for MaxMul).

Permutations and reshapes are data movement only (the plan's cuTENSOR step):
views where they can be, otherwise copies -- through the library's transpose
kernel when the permutation moves one group of adjacent axes past another,
through torch for other permutations and for tensors that need a gradient.
Every (+)/(x) runs in the HIP kernels.  Inside an
einsum, which operand is the GEMM's left one and the order of the contracted
labels are chosen so that the fewest elements are copied (an operand whose
permuted view is already contiguous costs nothing).  Gradients flow
through the library's autograd functions (float32/float64), so an einsum of
tensors that require grad is differentiable.
"""
from __future__ import annotations

import math
from typing import Iterable, Sequence

import torch

from . import ops

SEMIRINGS = ("maxplus", "minplus", "maxmul")
_ONE = {"maxplus": 0, "minplus": 0, "maxmul": 1}
_GRAD_DTYPES = (torch.float32, torch.float64)


def _check_semiring(semiring: str) -> None:
    if semiring not in SEMIRINGS:
        raise ValueError(f"unknown semiring {semiring!r}: expected one of {SEMIRINGS}")


def _needs_grad(*ts: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def _gemm(semiring: str, a: torch.Tensor, b: torch.Tensor, with_argmax: bool):
    """Row-major (batched) product of contiguous 2-D or 3-D tensors; through
    the autograd functions when a gradient is needed."""
    if _needs_grad(a, b):
        if with_argmax:
            raise ValueError("with_argmax=True is not available while recording gradients")
        if a.dtype not in _GRAD_DTYPES:
            raise RuntimeError(f"gradients are defined for float32/float64, got {a.dtype}")
        from . import pytorch as tp

        fn = {
            (2, "maxplus"): tp.TropicalMaxPlusMatmulGPU, (2, "minplus"): tp.TropicalMinPlusMatmulGPU,
            (2, "maxmul"): tp.TropicalMaxMulMatmulGPU,
            (3, "maxplus"): tp.TropicalMaxPlusMatmulBatched,
            (3, "minplus"): tp.TropicalMinPlusMatmulBatched,
            (3, "maxmul"): tp.TropicalMaxMulMatmulBatched,
        }[(a.dim(), semiring)]
        return fn.apply(a, b), None
    if a.dim() == 2:
        return ops.gemm(semiring, a.detach(), b.detach(), with_argmax)
    return ops.gemm_batched(semiring, a.detach(), b.detach(), with_argmax)


def _prod(sizes: Iterable[int]) -> int:
    return math.prod(sizes)


_TRANSPOSE_MAX_ROWS = (1 << 21) - 32  # tg_transpose's grid


def _layout(t: torch.Tensor, perm: list) -> torch.Tensor:
    """``t.permute(perm).contiguous()``.  A permutation that moves one group
    of adjacent axes past another -- a 2-D, or batched 2-D, transpose once the
    axes that stay together are merged -- runs through the library's
    transpose (``tg_transpose``); any other, and a tensor that needs a
    gradient, through torch."""
    v = t.permute(perm)
    if v.is_contiguous() or t.numel() == 0:
        return v.contiguous()
    if _needs_grad(t) or t.dtype not in ops._DT:
        return v.contiguous()
    if not t.is_contiguous():
        # A permuted view of a contiguous tensor (a contraction's result):
        # the same copy from that tensor's own layout.
        order = sorted(range(t.dim()), key=lambda d: -t.stride(d))
        base = t.permute(order)
        if not base.is_contiguous():
            return v.contiguous()
        pos = {a: i for i, a in enumerate(order)}
        return _layout(base, [pos[a] for a in perm])
    keep = [a for a in perm if t.shape[a] != 1]  # size-1 axes move no data
    order = sorted(keep)
    rank = {a: i for i, a in enumerate(order)}
    sizes = [t.shape[a] for a in order]  # the moved axes' sizes, in memory order
    groups = []  # runs of consecutive axes, in the order of the permuted view
    for a in (rank[x] for x in keep):
        if groups and groups[-1][-1] + 1 == a:
            groups[-1].append(a)
        else:
            groups.append([a])
    g = [_prod(sizes[a] for a in grp) for grp in groups]
    first = [grp[0] for grp in groups]
    if len(groups) == 2 and first[0] > first[1] and g[1] <= _TRANSPOSE_MAX_ROWS:
        out = ops.transpose(t.reshape(g[1], g[0]))  # [A, B] -> [B, A]
    elif len(groups) == 3 and first[0] < first[2] < first[1] and g[2] <= _TRANSPOSE_MAX_ROWS:
        out = ops.transpose(t.reshape(g[0], g[2], g[1]))  # [Z, A, B] -> [Z, B, A]
    else:
        return v.contiguous()
    return out.reshape(v.shape)


def _check_labels(name: str, t: torch.Tensor, labels: Sequence) -> None:
    if t.dim() != len(labels):
        raise ValueError(f"{name} has {t.dim()} dimensions but {len(labels)} labels {list(labels)}")
    if len(set(labels)) != len(labels):
        raise ValueError(f"{name} repeats a label in {list(labels)}; take the diagonal first "
                         "(einsum does this)")


def classify(ia: Sequence, ib: Sequence, iy: Sequence) -> dict:
    """Index classes of a binary contraction (design plan :262-279), each in
    order of first appearance: ``batch`` (both inputs and output), ``left``
    (A and output), ``right`` (B and output), ``contracted`` (both inputs,
    not output), ``a_sum`` / ``b_sum`` (one input only, not output)."""
    sa, sb, sy = set(ia), set(ib), set(iy)
    if len(sy) != len(iy):
        raise ValueError(f"output labels {list(iy)} repeat a label")
    missing = [x for x in iy if x not in sa and x not in sb]
    if missing:
        raise ValueError(f"output labels {missing} appear in neither operand")
    return {
        "batch": [x for x in ia if x in sb and x in sy],
        "left": [x for x in ia if x not in sb and x in sy],
        "right": [x for x in ib if x not in sa and x in sy],
        "contracted": [x for x in ia if x in sb and x not in sy],
        "a_sum": [x for x in ia if x not in sb and x not in sy],
        "b_sum": [x for x in ib if x not in sa and x not in sy],
    }


def _reduce(t: torch.Tensor, labels: list, drop: list, semiring: str):
    """Tropical sum of ``t`` over the labels in ``drop``: a product with a
    column of the semiring's one.  Returns the tensor and its labels."""
    if not drop:
        return t, list(labels)
    keep = [x for x in labels if x not in drop]
    perm = [labels.index(x) for x in keep] + [labels.index(x) for x in drop]
    keep_shape = [t.shape[labels.index(x)] for x in keep]
    rows = _prod(keep_shape)
    k = _prod(t.shape[labels.index(x)] for x in drop)
    mat = _layout(t, perm).reshape(rows, k)
    ones = torch.full((k, 1), _ONE[semiring], dtype=t.dtype, device=t.device)
    out, _ = _gemm(semiring, mat, ones, False)
    return out.reshape(keep_shape), keep


def contract_binary(a, b, ia: Sequence, ib: Sequence, iy: Sequence, semiring: str = "maxplus",
                    with_argmax: bool = False):
    """``Y[iy] = (+)_{contracted} A[ia] (x) B[ib]`` as one (batched) GEMM.

    Returns ``Y`` (and, with ``with_argmax``, an int32 tensor of Y's shape
    holding the row-major index over the contracted labels -- in their order
    of appearance in ``ia`` -- of the first term attaining each output; 0 when
    nothing is contracted).  Labels that appear in one operand only and not in
    the output are summed inside that operand first; their argmax is not
    tracked, so ``with_argmax`` requires that there are none."""
    return _contract(a, b, ia, ib, iy, semiring, with_argmax, False)


def _copy_cost(t: torch.Tensor, perm: list) -> int:
    """Elements copied to lay ``t`` out in the order ``perm`` (0 when the
    permuted view is already contiguous)."""
    return 0 if t.permute(perm).is_contiguous() else t.numel()


def _contract(a, b, ia, ib, iy, semiring, with_argmax, fewest_copies):
    """contract_binary; with ``fewest_copies`` the operand order and the order
    of the contracted labels (both free when no argmax is returned) are chosen
    to copy the fewest elements into GEMM layout."""
    _check_semiring(semiring)
    a = ops.as_tensor(a)
    b = ops.as_tensor(b)
    ia, ib, iy = list(ia), list(ib), list(iy)
    _check_labels("A", a, ia)
    _check_labels("B", b, ib)
    if a.dtype != b.dtype:
        raise ValueError(f"operands must have one dtype, got {a.dtype} and {b.dtype}")
    if a.device != b.device or a.device.type != "cuda":
        raise ValueError("operands must be device tensors on the same GPU")
    for x in set(ia) & set(ib):
        if a.shape[ia.index(x)] != b.shape[ib.index(x)]:
            raise ValueError(f"label {x!r} has size {a.shape[ia.index(x)]} in A and "
                             f"{b.shape[ib.index(x)]} in B")
    cls = classify(ia, ib, iy)
    if with_argmax and (cls["a_sum"] or cls["b_sum"]):
        raise ValueError("with_argmax needs every summed label to appear in both operands; "
                         f"{cls['a_sum'] + cls['b_sum']} appear in one only")
    a, ia = _reduce(a, ia, cls["a_sum"], semiring)
    b, ib = _reduce(b, ib, cls["b_sum"], semiring)
    size = {x: a.shape[ia.index(x)] for x in ia}
    size.update({x: b.shape[ib.index(x)] for x in ib})

    batch, left, right, con = cls["batch"], cls["left"], cls["right"], cls["contracted"]
    if fewest_copies:
        # Candidates: (swap operands?, contracted-label order); the first one
        # is the documented layout, kept on ties.
        cands = []
        for swap in (False, True):
            x, lx, y, ly = (b, ib, a, ia) if swap else (a, ia, b, ib)
            lft, rgt = (right, left) if swap else (left, right)
            orders = []
            for o in (con, [c for c in lx if c in con], [c for c in ly if c in con]):
                if o not in orders:
                    orders.append(o)
            for order in orders:
                cost = (_copy_cost(x, [lx.index(c) for c in batch + lft + order]) +
                        _copy_cost(y, [ly.index(c) for c in batch + order + rgt]))
                cands.append((cost, len(cands), swap, order))
        _, _, swap, con = min(cands)
        if swap:
            a, ia, b, ib = b, ib, a, ia
            left, right = right, left
    nb = _prod(size[x] for x in batch)
    m = _prod(size[x] for x in left)
    n = _prod(size[x] for x in right)
    k = _prod(size[x] for x in con)  # 1 when nothing is contracted (outer product)
    am = _layout(a, [ia.index(x) for x in batch + left + con])
    bm = _layout(b, [ib.index(x) for x in batch + con + right])
    if batch:
        c, idx = _gemm(semiring, am.reshape(nb, m, k), bm.reshape(nb, k, n), with_argmax)
    else:
        c, idx = _gemm(semiring, am.reshape(m, k), bm.reshape(k, n), with_argmax)
    order = batch + left + right
    shape = [size[x] for x in order]
    perm = [order.index(x) for x in iy]
    y = c.reshape(shape).permute(perm)
    if not with_argmax:
        return y
    return y, idx.reshape(shape).permute(perm)


# ---------------------------------------------------------------------------
# Einsum engine
# ---------------------------------------------------------------------------

def parse(code: str, nops: int | None = None):
    """``"ij,jk->ik"`` -> ``([['i','j'], ['j','k']], ['i','k'])``.  Labels are
    letters; without ``->`` the output is every label that appears exactly
    once, in alphabetical order (numpy's implicit mode)."""
    code = code.replace(" ", "")
    if "." in code:
        raise ValueError("ellipsis ('...') is not supported")
    if "->" in code:
        lhs, rhs = code.split("->")
        if "->" in rhs:
            raise ValueError(f"einsum code {code!r} has more than one '->'")
    else:
        lhs, rhs = code, None
    ixs = [list(term) for term in lhs.split(",")]
    for term in ixs + ([list(rhs)] if rhs is not None else []):
        for ch in term:
            if not ch.isalpha():
                raise ValueError(f"invalid label {ch!r} in einsum code {code!r}")
    if rhs is None:
        counts = {}
        for term in ixs:
            for ch in term:
                counts[ch] = counts.get(ch, 0) + 1
        iy = sorted(ch for ch, c in counts.items() if c == 1)
    else:
        iy = list(rhs)
    if nops is not None and len(ixs) != nops:
        raise ValueError(f"einsum code {code!r} names {len(ixs)} operands, got {nops}")
    return ixs, iy


def _pair_result(li: list, lj: list, keep: set) -> list:
    """Labels of the result of contracting operands with labels li and lj
    when the labels in ``keep`` are still needed (output or other operands)."""
    out = []
    for x in li + lj:
        if x in keep and x not in out:
            out.append(x)
    return out


def einsum_path(ixs: Sequence[Sequence], iy: Sequence, sizes: dict, optimize="greedy"):
    """Pairwise contraction order: a list of ``(i, j)`` positions into the
    current operand list; the pair is removed and its result appended.

    ``optimize="greedy"`` picks, at every step, the pair whose result has
    the fewest elements (ties: fewer terms, i.e. a smaller product of all
    the pair's label sizes, then the first pair in list order) -- the plan's
    ``GreedyMethod::new(0.0, 0.0)``.  ``optimize=None`` contracts left to
    right."""
    ops_ = [list(x) for x in ixs]
    path = []
    while len(ops_) > 1:
        if optimize is None or optimize is False:
            i, j = 0, 1
        elif optimize == "greedy":
            best = None
            for i_ in range(len(ops_)):
                for j_ in range(i_ + 1, len(ops_)):
                    keep = set(iy)
                    for o, lab in enumerate(ops_):
                        if o not in (i_, j_):
                            keep.update(lab)
                    res = _pair_result(ops_[i_], ops_[j_], keep)
                    cost = (_prod(sizes[x] for x in res),
                            _prod(sizes[x] for x in set(ops_[i_]) | set(ops_[j_])), i_, j_)
                    if best is None or cost < best[0]:
                        best = (cost, i_, j_)
            _, i, j = best
        else:
            raise ValueError(f"unknown optimize={optimize!r}: expected 'greedy' or None")
        keep = set(iy)
        for o, lab in enumerate(ops_):
            if o not in (i, j):
                keep.update(lab)
        res = _pair_result(ops_[i], ops_[j], keep)
        path.append((i, j))
        ops_ = [lab for o, lab in enumerate(ops_) if o not in (i, j)] + [res]
    return path


def _diagonal(t: torch.Tensor, labels: list):
    """Take the diagonal over every repeated label of one operand."""
    labels = list(labels)
    while len(set(labels)) != len(labels):
        seen = {}
        for p, x in enumerate(labels):
            if x in seen:
                q = seen[x]
                if t.shape[q] != t.shape[p]:
                    raise ValueError(f"repeated label {x!r} has sizes {t.shape[q]} and {t.shape[p]}")
                t = torch.diagonal(t, dim1=q, dim2=p)  # the diagonal moves to the last axis
                labels = [y for r, y in enumerate(labels) if r not in (q, p)] + [x]
                break
            seen[x] = p
    return t, labels


def einsum(code: str, *operands, semiring: str = "maxplus", optimize="greedy") -> torch.Tensor:
    """Tropical einsum over device tensors, e.g.
    ``einsum("ijk,jkl,lm->im", a, b, c, semiring="maxplus")``.

    Every operand must be a device tensor of one dtype (float32, float64,
    int32 or int64).  Returns a new tensor (a view for a pure permutation of
    one operand).  Differentiable for float tensors that require grad."""
    _check_semiring(semiring)
    if not operands:
        raise ValueError("einsum needs at least one operand")
    ts = [ops.as_tensor(t) for t in operands]
    ixs, iy = parse(code, len(ts))
    dt, dev = ts[0].dtype, ts[0].device
    for p, t in enumerate(ts):
        if t.dtype != dt or t.device != dev:
            raise ValueError(f"operand {p} is {t.dtype} on {t.device}; operand 0 is {dt} on {dev}")
        if t.dim() != len(ixs[p]):
            raise ValueError(f"operand {p} has {t.dim()} dimensions but {len(ixs[p])} labels")
    if dev.type != "cuda":
        raise ValueError("einsum needs device tensors; move the operands to the GPU first")
    sizes: dict = {}
    for t, lab in zip(ts, ixs):
        for x, s in zip(lab, t.shape):
            if sizes.setdefault(x, s) != s:
                raise ValueError(f"label {x!r} has sizes {sizes[x]} and {s}")
    if len(set(iy)) != len(iy):
        raise ValueError(f"output labels {iy} repeat a label")
    missing = [x for x in iy if x not in sizes]
    if missing:
        raise ValueError(f"output labels {missing} appear in no operand")

    # Diagonals, then labels summed inside one operand (nowhere else, not in
    # the output).
    cur = []
    for p, (t, lab) in enumerate(zip(ts, ixs)):
        t, lab = _diagonal(t, lab)
        others = set(iy)
        for q, lq in enumerate(ixs):
            if q != p:
                others.update(lq)
        t, lab = _reduce(t, lab, [x for x in lab if x not in others], semiring)
        cur.append((t, lab))

    for i, j in einsum_path([lab for _, lab in cur], iy, sizes, optimize):
        keep = set(iy)
        for o, (_, lab) in enumerate(cur):
            if o not in (i, j):
                keep.update(lab)
        (ta, la), (tb, lb) = cur[i], cur[j]
        res = _pair_result(la, lb, keep)
        tc = _contract(ta, tb, la, lb, res, semiring, False, True)
        cur = [c for o, c in enumerate(cur) if o not in (i, j)] + [(tc, res)]

    t, lab = cur[0]
    return t.permute([lab.index(x) for x in iy])


__all__ = ["classify", "contract_binary", "einsum", "einsum_path", "parse", "SEMIRINGS"]
