"""GPU backward (argmax scatter) and the PyTorch autograd mirror.

The reference accumulates grad_A[i, argmax[i,j]] += dC[i,j] and
grad_B[argmax[i,j], j] += dC[i,j] visiting i then j ascending
(crates/tropical-gemm/src/api.rs:563-582, 627-646), and the oracle restates
that loop.  The HIP kernels reproduce the order of every sum
(tg_backward.hpp), so gradients must equal the oracle bit for bit, for f32 and
f64, on every argmax pattern, and be identical from run to run.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def assert_bits(got, ref):
    np.testing.assert_array_equal(tc.bits(np.ascontiguousarray(got)), tc.bits(np.ascontiguousarray(ref)))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
@pytest.mark.parametrize("shape", [(37, 23, 29), (130, 300, 70), (5, 1, 9), (64, 9000, 3),
                                   (3, 40000, 5), (200, 128, 700)])
def test_backward_matches_oracle(dtype, sr, shape):
    from tropical_gemm import ops

    m, k, n = shape
    rng = np.random.default_rng(21)
    a = rng.standard_normal((m, k)).astype(dtype)
    b = rng.standard_normal((k, n)).astype(dtype)
    g = rng.standard_normal((m, n)).astype(dtype)
    _, am = oracle.gemm(sr, a, b)
    mult = sr == "maxmul"
    ta, tb, tg = (torch.from_numpy(x).to(DEV) for x in (a, b, g))
    tam = torch.from_numpy(am.astype(np.int32)).to(DEV)
    ga = ops.backward_a(tg, tam, k, b=tb if mult else None).cpu().numpy()
    gb = ops.backward_b(tg, tam, k, a=ta if mult else None).cpu().numpy()
    assert_bits(ga, oracle.backward_a(g, am, k, b if mult else None))
    assert_bits(gb, oracle.backward_b(g, am, k, a if mult else None))


# Argmax patterns that steer the LDS-bin kernels down each of their paths:
# spread indices (lanes alone with their bin: a plain read-add-write), paired
# and clustered indices (shared bins: ordered LDS float atomics), one or four
# bins per block (rows and columns on atomics alone), and the argmax of
# N(0,1) data (about half the lanes of a block share a bin).
PATTERNS = ["uniform", "all zero", "four values", "k = j", "pairs", "row argmax"]
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("pattern", PATTERNS)
def test_backward_index_patterns(dtype, pattern):
    from tropical_gemm import ops

    m, n, k = 192, 1024, 1024
    rng = np.random.default_rng(23 + PATTERNS.index(pattern))
    g = rng.standard_normal((m, n)).astype(dtype)
    if pattern == "uniform":
        am = rng.integers(0, k, size=(m, n))
    elif pattern == "all zero":
        am = np.zeros((m, n), np.int64)
    elif pattern == "four values":
        am = rng.integers(0, 4, size=(m, n))
    elif pattern == "k = j":
        am = np.tile(np.arange(n), (m, 1))
    elif pattern == "pairs":  # lanes 2t and 2t+1 share an index
        am = np.repeat(rng.integers(0, k, size=(m, n // 2)), 2, axis=1)
    else:  # the argmax of N(0,1) data: a few hundred distinct k per row
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        _, am = oracle.gemm("maxplus", a, b)
    am = am.astype(np.int64)
    print(f"[case] backward pattern {pattern} {np.dtype(dtype).name}", flush=True)
    tg = torch.from_numpy(g).to(DEV)
    tam = torch.from_numpy(am.astype(np.int32)).to(DEV)
    ga = ops.backward_a(tg, tam, k).cpu().numpy()
    gb = ops.backward_b(tg, tam, k).cpu().numpy()
    assert_bits(ga, oracle.backward_a(g, am.astype(np.uint32), k))
    assert_bits(gb, oracle.backward_b(g, am.astype(np.uint32), k))
    # Run to run: the same bits again.
    assert_bits(ops.backward_a(tg, tam, k).cpu().numpy(), ga)
    assert_bits(ops.backward_b(tg, tam, k).cpu().numpy(), gb)


# Sums whose bits depend on every rounding step, on the LDS-bin kernels
# (ordered LDS float atomics where lanes of a block share a bin, a plain
# read-add-write where a lane is alone with it): contributions of mixed
# magnitudes (2^-30 .. 2^30), round-to-even ties (1.0 among halves of an
# ulp), denormal values and cancellations into the denormal range.  Rows
# (and columns) whose first block is one bin run on atomics alone, the others
# count first: rows 0 mod 3 start with a one-bin block and then spread, rows
# 1 mod 3 start spread and then use three bins, and the first 64 rows of
# every fifth column are one bin.
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_backward_rounding_denormals_and_modes(dtype):
    from tropical_gemm import ops

    m, n, k = 160, 2048, 512
    rng = np.random.default_rng(77)
    fi = np.finfo(dtype)
    g = rng.standard_normal((m, n)) * np.exp2(rng.integers(-30, 31, size=(m, n)))
    g[:48] = np.where(rng.random((48, n)) < 0.1, 1.0,
                      fi.eps / 2 * rng.integers(1, 4, size=(48, n)) * rng.choice([-1, 1], size=(48, n)))
    g[48:96] = rng.uniform(0.5, 1, size=(48, n)) * rng.choice([-1, 1], size=(48, n)) * float(
        fi.tiny) * np.exp2(rng.integers(-20, 4, size=(48, n)))
    g = g.astype(dtype)
    assert (np.abs(g[48:96]) < fi.tiny).any() and (g[48:96] != 0).all()  # denormal contributions
    am = rng.integers(0, k, size=(m, n))
    for i in range(m):
        if i % 3 == 0:
            am[i, :64] = 7
        elif i % 3 == 1:
            am[i, 64:] = rng.integers(0, 3, size=n - 64)
    am[:64, ::5] = 11
    print(f"[case] backward rounding/denormals {np.dtype(dtype).name}", flush=True)
    tg = torch.from_numpy(g).to(DEV)
    tam = torch.from_numpy(am.astype(np.int32)).to(DEV)
    ga = ops.backward_a(tg, tam, k).cpu().numpy()
    gb = ops.backward_b(tg, tam, k).cpu().numpy()
    ref_a = oracle.backward_a(g, am.astype(np.uint32), k)
    ref_b = oracle.backward_b(g, am.astype(np.uint32), k)
    assert ((np.abs(ref_a[48:96]) < fi.tiny) & (ref_a[48:96] != 0)).any()  # denormal sums
    assert_bits(ga, ref_a)
    assert_bits(gb, ref_b)


def test_backward_column_major_and_out_of_range_index():
    from tropical_gemm import _native as nat

    lib = nat.load()
    m, k, n = 6, 4, 5
    rng = np.random.default_rng(2)
    g = rng.standard_normal((m, n)).astype(np.float32)
    am = rng.integers(0, k, size=(m, n)).astype(np.int32)
    am[0, 0] = k + 3   # skipped (tropical_gemm.cu:1014, api.rs:575-582)
    am[1, 1] = -1      # skipped
    ref_a = oracle.backward_a(g, np.where(am < 0, 10**6, am).astype(np.uint32), k)
    ref_b = oracle.backward_b(g, np.where(am < 0, 10**6, am).astype(np.uint32), k)
    # Column-major storage of g / argmax; outputs come back column-major.
    tg = torch.from_numpy(g.T.copy()).to(DEV)
    tam = torch.from_numpy(am.T.copy()).to(DEV)
    ga = torch.empty(m * k, dtype=torch.float32, device=DEV)
    gb = torch.empty(k * n, dtype=torch.float32, device=DEV)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    nat.check(lib.tg_backward_a(0, 0, 1, p(tg), p(tam), p(ga), m, n, k, None))
    nat.check(lib.tg_backward_b(0, 0, 1, p(tg), p(tam), p(gb), m, n, k, None))
    torch.cuda.synchronize()
    assert_bits(ga.cpu().numpy().reshape(k, m).T, ref_a)
    assert_bits(gb.cpu().numpy().reshape(n, k).T, ref_b)


# Products with no rows or no columns: every gradient element has no
# contribution, so each gradient comes back all +0 (the reference's zeroed
# output, api.rs:563-582), with NULL grad_c / argmax (and NULL `other`)
# accepted.  The scatter kernels must not run: their first clamped read would
# be at index -1.
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("mult", [False, True])
@pytest.mark.parametrize("shape", [(37, 0, 29), (0, 23, 29)])
@pytest.mark.parametrize("layout", [0, 1])
def test_backward_empty_product(dtype, mult, shape, layout):
    from tropical_gemm import _native as nat

    lib = nat.load()
    m, n, k = shape
    dt = 0 if dtype == np.float32 else 1
    print(f"[case] backward empty m={m} n={n} k={k} {np.dtype(dtype).name} mult={mult} layout={layout}",
          flush=True)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    tdt = torch.float32 if dtype == np.float32 else torch.float64
    for want_a, elems in ((True, m * k), (False, k * n)):
        if elems == 0:
            continue
        out = torch.full((elems + 8,), float("nan"), dtype=tdt, device=DEV)
        if mult:
            fn = lib.tg_maxmul_backward_a if want_a else lib.tg_maxmul_backward_b
            nat.check(fn(0, dt, layout, None, None, None, p(out), m, n, k, None))
        else:
            fn = lib.tg_backward_a if want_a else lib.tg_backward_b
            nat.check(fn(0, dt, layout, None, None, p(out), m, n, k, None))
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert_bits(got[:elems], np.zeros(elems, dtype))
        assert np.all(np.isnan(got[elems:])), "wrote past the gradient"
    # Strided batches with gaps: every matrix zeroed, the gaps untouched.
    batch = 3
    for want_a, elems in ((True, m * k), (False, k * n)):
        if elems == 0:
            continue
        stride = elems + 5
        out = torch.full((batch * stride,), float("nan"), dtype=tdt, device=DEV)
        fn = lib.tg_backward_a_strided_batched if want_a else lib.tg_backward_b_strided_batched
        nat.check(fn(0, dt, layout, None, None, None, p(out), batch, m, n, k, m * n,
                     k * n if want_a else m * k, stride, None))
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(batch, stride)
        assert_bits(got[:, :elems], np.zeros((batch, elems), dtype))
        assert np.all(np.isnan(got[:, elems:]))


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_batched_backward(sr):
    from tropical_gemm import ops

    rng = np.random.default_rng(31)
    batch, m, k, n = 3, 20, 17, 11
    a = rng.standard_normal((batch, m, k)).astype(np.float32)
    b = rng.standard_normal((batch, k, n)).astype(np.float32)
    g = rng.standard_normal((batch, m, n)).astype(np.float32)
    mult = sr == "maxmul"
    ta, tb, tg = (torch.from_numpy(x).to(DEV) for x in (a, b, g))
    _, tam = ops.gemm_batched(sr, ta, tb, True)
    ga = ops.backward_a_batched(tg, tam, k, b=tb if mult else None).cpu().numpy()
    gb = ops.backward_b_batched(tg, tam, k, a=ta if mult else None).cpu().numpy()
    am = tam.cpu().numpy()
    for t in range(batch):
        _, am_ref = oracle.gemm(sr, a[t], b[t])
        np.testing.assert_array_equal(am[t], am_ref.astype(np.int32))
        assert_bits(ga[t], oracle.backward_a(g[t], am_ref, k, b[t] if mult else None))
        assert_bits(gb[t], oracle.backward_b(g[t], am_ref, k, a[t] if mult else None))


# ---------------------------------------------------------------------------
# Autograd mirror (reference pytorch.py GPU classes)
# ---------------------------------------------------------------------------

def _scatter_reference(a, b, argmax, grad_c, mult):
    """The reference's own backward (pytorch.py:386-403, 521-548) in float64 on CPU."""
    a, b, argmax, grad_c = (x.detach().double().cpu() if x.is_floating_point() else x.cpu()
                            for x in (a, b, argmax, grad_c))
    argmax = argmax.long()
    m, k = a.shape
    n = b.shape[1]
    if mult:
        b_win = b[argmax, torch.arange(n).unsqueeze(0).expand(m, -1)]
        a_win = torch.gather(a, 1, argmax)
        ga = torch.zeros(m, k, dtype=torch.float64).scatter_add_(1, argmax, grad_c * b_win)
        gbt = torch.zeros(n, k, dtype=torch.float64).scatter_add_(1, argmax.t(), (grad_c * a_win).t())
    else:
        ga = torch.zeros(m, k, dtype=torch.float64).scatter_add_(1, argmax, grad_c)
        gbt = torch.zeros(n, k, dtype=torch.float64).scatter_add_(1, argmax.t(), grad_c.t())
    return ga, gbt.t()


@pytest.mark.parametrize("name", ["maxplus", "minplus", "maxmul"])
def test_autograd_gpu_classes(name):
    from tropical_gemm import pytorch as tp

    fn = {"maxplus": tp.tropical_maxplus_matmul_gpu, "minplus": tp.tropical_minplus_matmul_gpu,
          "maxmul": tp.tropical_maxmul_matmul_gpu}[name]
    g = torch.Generator(device="cpu").manual_seed(5)
    a = torch.randn(50, 40, generator=g).to(DEV).requires_grad_(True)
    b = torch.randn(40, 30, generator=g).to(DEV).requires_grad_(True)
    c = fn(a, b)
    c_ref, am_ref = oracle.gemm(name, a.detach().cpu().numpy(), b.detach().cpu().numpy())
    np.testing.assert_array_equal(c.detach().cpu().numpy(), c_ref)
    grad_c = torch.randn(50, 30, generator=g).to(DEV)
    c.backward(grad_c)
    # References from the oracle's argmax, never the GPU's: the reference's
    # own scatter_add_ formulation (float64) and the oracle's loop (bit for bit).
    argmax = torch.from_numpy(am_ref.astype(np.int64))
    mult = name == "maxmul"
    ga_ref, gb_ref = _scatter_reference(a, b, argmax, grad_c, mult)
    torch.testing.assert_close(a.grad.double().cpu(), ga_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(b.grad.double().cpu(), gb_ref, rtol=1e-5, atol=1e-5)
    an, bn, gn = (x.detach().cpu().numpy() for x in (a, b, grad_c))
    assert_bits(a.grad.cpu().numpy(), oracle.backward_a(gn, am_ref, 40, bn if mult else None))
    assert_bits(b.grad.cpu().numpy(), oracle.backward_b(gn, am_ref, 40, an if mult else None))


def test_autograd_finite_differences_maxplus():
    # Structure of crates/tropical-gemm-cuda/src/lib.rs:1265-1330 (eps 1e-3, tol 0.05).
    from tropical_gemm import pytorch as tp

    m, k, n = 4, 5, 3
    a = torch.tensor([[(i * k + kk) * 0.7 - 3.0 for kk in range(k)] for i in range(m)],
                     dtype=torch.float64, device=DEV, requires_grad=True)
    b = torch.tensor([[(kk * n + j) * 0.5 - 2.0 for j in range(n)] for kk in range(k)],
                     dtype=torch.float64, device=DEV, requires_grad=True)
    c = tp.tropical_maxplus_matmul_gpu(a, b)
    for i in range(m):
        for j in range(n):
            ga, = torch.autograd.grad(c[i, j], a, retain_graph=True)
            for kk in range(k):
                ap = a.detach().clone()
                ap[i, kk] += 1e-3
                num = (tp.tropical_maxplus_matmul_gpu(ap, b.detach())[i, j] - c[i, j].detach()) / 1e-3
                assert abs(float(num) - float(ga[i, kk])) < 0.05


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_autograd_finite_differences_maxmul(dtype):
    """MaxMul rule (grad_A += dC * B[argmax, j], grad_B += dC * A[i, argmax])
    against central differences, on the operands of the reference's own test
    (test_pytorch_gradients.py:279-334: well-separated values so no argmax
    flips under eps) in f32 and f64, and on a random positive 6 x 5 x 4
    problem in f64."""
    from tropical_gemm import pytorch as tp

    f = tp.tropical_maxmul_matmul_gpu
    g = torch.Generator(device="cpu").manual_seed(9)
    cases = [
        (torch.tensor([[1.0, 10.0], [8.0, 1.0]]), torch.tensor([[1.0, 1.0], [2.0, 3.0]])),
        (torch.rand(6, 5, generator=g) * 4 + 1, torch.rand(5, 4, generator=g) * 4 + 1),
    ]
    eps = 1e-4 if dtype == torch.float32 else 1e-6
    if dtype == torch.float32:
        cases = cases[:1]  # f32 central differences of a 6 x 4 sum are too coarse at eps 1e-4
    for a0, b0 in cases:
        a = a0.to(DEV, dtype).requires_grad_(True)
        b = b0.to(DEV, dtype).requires_grad_(True)
        f(a, b).sum().backward()
        for x, other, grad, left in ((a, b, a.grad, True), (b, a, b.grad, False)):
            num = torch.zeros_like(x)
            for idx in np.ndindex(*x.shape):
                xp, xm = x.detach().clone(), x.detach().clone()
                xp[idx] += eps
                xm[idx] -= eps
                cp = f(xp, other.detach()) if left else f(other.detach(), xp)
                cm = f(xm, other.detach()) if left else f(other.detach(), xm)
                num[idx] = (cp.sum() - cm.sum()) / (2 * eps)
            assert torch.allclose(grad, num, atol=0.1), (grad, num)


def test_backward_rows_beyond_2_24():
    """grad_A of a 2^24 + 1 row problem (K = 3, N = 2): more rows than one
    launch dimension of 256-thread workgroups could hold; the kernel loops
    over rows with a capped grid (tg_backward_plan)."""
    from tropical_gemm import _native as nat, ops

    m, n, k = (1 << 24) + 1, 2, 3
    plan = nat.load().tg_backward_plan(0, 0, 1, 1, m, n, k).decode()
    print(f"[case] backward rows {m}x{n}x{k}: {plan}", flush=True)
    assert "grid=16384" in plan
    rng = np.random.default_rng(77)
    g = rng.standard_normal((m, n)).astype(np.float32)
    am = rng.integers(0, k, size=(m, n)).astype(np.int32)
    am[0, 0] = -1
    am[m - 1, 1] = k  # out of range: skipped
    tg_, tam = torch.from_numpy(g).to(DEV), torch.from_numpy(am).to(DEV)
    ga = ops.backward_a(tg_, tam, k).cpu().numpy()
    ref = oracle.backward_a(g, np.where(am < 0, 1 << 30, am).astype(np.uint32), k)
    assert_bits(ga, ref)


def test_backward_cols_tall_skinny():
    """grad_B with few columns and many rows: each bin is one long ordered
    chain (K = 3 bins per column), which takes the serial per-bin path."""
    from tropical_gemm import ops

    m, n, k = 1 << 18, 2, 3
    rng = np.random.default_rng(78)
    g = rng.standard_normal((m, n)).astype(np.float32)
    am = rng.integers(0, k, size=(m, n)).astype(np.int32)
    tg_, tam = torch.from_numpy(g).to(DEV), torch.from_numpy(am).to(DEV)
    gb = ops.backward_b(tg_, tam, k).cpu().numpy()
    assert_bits(gb, oracle.backward_b(g, am.astype(np.uint32), k))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("k", [70000, 40000])
def test_backward_bins_in_global_memory(dtype, k):
    """K too large for LDS bins (f32 K = 70000: 273 KB per row): the bins are
    the gradient itself, same order, same bits."""
    from tropical_gemm import _native as nat, ops

    m, n = 5, 3000
    dt = 0 if dtype == np.float32 else 1
    plan_a = nat.load().tg_backward_plan(dt, 0, 1, 1, m, n, k).decode()
    plan_b = nat.load().tg_backward_plan(dt, 0, 0, 1, m, n, k).decode()
    print(f"[case] global bins {np.dtype(dtype).name} k={k}: {plan_a} / {plan_b}", flush=True)
    if k * np.dtype(dtype).itemsize > 128 * 1024:
        # grad_B: global bins, or eight columns in passes over the keys.
        assert "global" in plan_a and ("global" in plan_b or "passes=" in plan_b)
    rng = np.random.default_rng(k)
    g = rng.standard_normal((m, n)).astype(dtype)
    am = rng.integers(0, k, size=(m, n)).astype(np.int32)
    am[:, :200] = 7  # one bin repeated across whole blocks
    tg_, tam = torch.from_numpy(g).to(DEV), torch.from_numpy(am).to(DEV)
    assert_bits(ops.backward_a(tg_, tam, k).cpu().numpy(), oracle.backward_a(g, am.astype(np.uint32), k))
    assert_bits(ops.backward_b(tg_, tam, k).cpu().numpy(), oracle.backward_b(g, am.astype(np.uint32), k))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("gap", [0, 1000])
def test_backward_b_global_bins_batched(dtype, gap):
    """grad_B with its bins in global memory on a strided batch, dense
    (gap 0) or with `gap` elements between the items: the gradient is
    zero-filled item by item before the scatter, and the gaps keep their
    bytes."""
    from tropical_gemm import _native as nat

    lib = nat.load()
    batch, m, n, k = 3, 7, 130, 70000
    dt = 0 if dtype == np.float32 else 1
    plan = lib.tg_backward_plan(dt, 0, 0, batch, m, n, k).decode()
    print(f"[case] grad_B global bins batched {np.dtype(dtype).name} gap={gap}: {plan}", flush=True)
    assert plan.startswith("cols global"), plan
    rng = np.random.default_rng(4000 + gap)
    g = rng.standard_normal((batch, m, n)).astype(dtype)
    am = rng.integers(0, k, size=(batch, m, n))
    am[:, :, :40] = 5  # one bin repeated within blocks
    am[0, 0, 0], am[1, 2, 3] = -1, k  # skipped
    s_b = k * n + gap
    out = torch.full((batch * s_b,), 7.0, dtype=torch.float32 if dt == 0 else torch.float64, device=DEV)
    tg_ = torch.from_numpy(g).to(DEV)
    tam = torch.from_numpy(am.astype(np.int32)).to(DEV)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    nat.check(lib.tg_backward_b_strided_batched(0, dt, 0, p(tg_), p(tam), None, p(out), batch, m, n, k,
                                                m * n, 0, s_b, None))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for t in range(batch):
        ref = oracle.backward_b(g[t], np.where(am[t] < 0, 1 << 30, am[t]).astype(np.uint32), k)
        assert_bits(got[t * s_b:t * s_b + k * n].reshape(k, n), ref)
        assert (got[t * s_b + k * n:(t + 1) * s_b] == 7.0).all()


# grad_B with columns too long for eight columns' bins in the LDS: few rows
# take the keys in passes over eight columns (the planner's pass length is
# what the LDS holds: 4288 keys f32, 1872 f64), many rows fewer columns per
# workgroup in one pass.  Cases: dtype, K, M, a fragment of the plan, MaxMul.
LONG_COLUMNS = [
    (np.float32, 8192, 300, "passes=2", False), (np.float32, 8192, 300, "passes=2", True),
    (np.float32, 32768, 300, "passes=8", True), (np.float32, 40000, 60, "passes=10", False),
    (np.float64, 16384, 300, "passes=9", True),
    (np.float32, 8192, 4500, "waves=4 ", False), (np.float32, 12000, 4500, "waves=3 ", False),
    (np.float32, 16384, 4500, "waves=2 ", False), (np.float32, 32768, 4500, "waves=1 ", False),
    (np.float64, 4096, 4500, "waves=4 ", False), (np.float64, 16384, 4500, "waves=1 ", False),
]


@pytest.mark.parametrize("dtype,k,m,frag,mult", LONG_COLUMNS,
                         ids=[f"{np.dtype(c[0]).name}-k{c[1]}-m{c[2]}-{c[3].strip()}{'-maxmul' if c[4] else ''}"
                              for c in LONG_COLUMNS])
def test_backward_cols_long_columns_in_lds(dtype, k, m, frag, mult):
    """grad_B with long columns whose bins live in the LDS: keys on the
    edges of the passes, a column group that ends past N, rows that end
    inside a tile, bins repeated within blocks and out-of-range indices must
    still give the reference's bits."""
    from tropical_gemm import _native as nat, ops

    n = 21
    dt = 0 if dtype == np.float32 else 1
    plan = nat.load().tg_backward_plan(dt, 0, 0, 1, m, n, k).decode()
    print(f"[case] grad_B long columns {np.dtype(dtype).name} m={m} k={k} mult={mult}: {plan}", flush=True)
    assert plan.startswith("cols lds") and frag in plan, plan
    kp = 4288 if dtype == np.float32 else 1872
    edges = [e for p_ in range(1, 12) for e in (p_ * kp - 1, p_ * kp) if e < k] + [0, 1, k - 2, k - 1]
    rng = np.random.default_rng(k + m)
    g = rng.standard_normal((m, n)).astype(dtype)
    am = rng.integers(0, k, size=(m, n))
    am[:min(m, 96)] = rng.choice(edges, size=(min(m, 96), n))  # pass edges, repeated within blocks
    am[200:264, ::3] = k // 3  # one bin for a whole block (where the rows exist)
    am[5, 2], am[m - 1, 4], am[m - 1, n - 1] = -1, k, k + 5  # skipped
    a = rng.standard_normal((m, k)).astype(dtype) if mult else None
    tg_, tam = torch.from_numpy(g).to(DEV), torch.from_numpy(am.astype(np.int32)).to(DEV)
    ta = torch.from_numpy(a).to(DEV) if mult else None
    gb = ops.backward_b(tg_, tam, k, a=ta).cpu().numpy()
    ref = oracle.backward_b(g, np.where(am < 0, 1 << 30, am).astype(np.uint32), k, a)
    assert_bits(gb, ref)


@pytest.mark.parametrize("name", ["maxplus", "minplus", "maxmul"])
def test_autograd_batched_classes(name):
    from tropical_gemm import pytorch as tp

    fn = {"maxplus": tp.tropical_maxplus_matmul_batched,
          "minplus": tp.tropical_minplus_matmul_batched,
          "maxmul": tp.tropical_maxmul_matmul_batched}[name]
    g = torch.Generator(device="cpu").manual_seed(6)
    a = torch.randn(3, 12, 9, generator=g).to(DEV).requires_grad_(True)
    b = torch.randn(3, 9, 7, generator=g).to(DEV).requires_grad_(True)
    c = fn(a, b)
    c.sum().backward()
    for t in range(3):
        c_ref, am_ref = oracle.gemm(name, a[t].detach().cpu().numpy(), b[t].detach().cpu().numpy())
        np.testing.assert_array_equal(c[t].detach().cpu().numpy(), c_ref)
        am_t = torch.from_numpy(am_ref.astype(np.int64))
        ga_ref, gb_ref = _scatter_reference(a[t], b[t], am_t, torch.ones(12, 7), name == "maxmul")
        torch.testing.assert_close(a.grad[t].double().cpu(), ga_ref, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(b.grad[t].double().cpu(), gb_ref, rtol=1e-5, atol=1e-5)
    # Sum invariant for the additive rule (test_pytorch_gradients.py:515-518).
    if name != "maxmul":
        assert abs(float(a.grad.sum()) - 3 * 12 * 7) < 1e-3
        assert abs(float(b.grad.sum()) - 3 * 12 * 7) < 1e-3


def test_dlpack_and_numpy_faces():
    import tropical_gemm as tgm

    rng = np.random.default_rng(17)
    a = rng.standard_normal((13, 21)).astype(np.float32)
    b = rng.standard_normal((21, 8)).astype(np.float32)
    c_ref, am_ref = oracle.gemm("maxplus", a, b)
    ta, tb = torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV)
    c_cap, am_cap = tgm.maxplus_matmul_dlpack(ta, tb)
    c = torch.from_dlpack(c_cap).reshape(13, 8)
    am = torch.from_dlpack(am_cap).reshape(13, 8).to(torch.int64)
    np.testing.assert_array_equal(c.cpu().numpy(), c_ref)
    np.testing.assert_array_equal(am.cpu().numpy(), am_ref)
    # numpy face: row-major correct for non-square inputs.
    c_np, am_np = tgm.maxplus_matmul_gpu_with_argmax(a, b)
    np.testing.assert_array_equal(c_np.reshape(13, 8), c_ref)
    np.testing.assert_array_equal(am_np.reshape(13, 8), am_ref.astype(np.int32))
    np.testing.assert_array_equal(tgm.minplus_matmul_gpu(a, b).reshape(13, 8),
                                  oracle.gemm("minplus", a, b, with_argmax=False)[0])
    with pytest.raises(ValueError, match="Zero-sized"):
        tgm.maxplus_matmul_dlpack(torch.zeros(0, 3, device=DEV), torch.zeros(3, 2, device=DEV))
    with pytest.raises(ValueError, match="same dtype"):
        tgm.maxplus_matmul_dlpack(ta, tb.double())
    a3 = torch.from_numpy(rng.standard_normal((2, 5, 6)).astype(np.float32)).to(DEV)
    b3 = torch.from_numpy(rng.standard_normal((2, 6, 4)).astype(np.float32)).to(DEV)
    c_cap, am_cap = tgm.maxmul_matmul_batched_dlpack(a3, b3)
    c3 = torch.from_dlpack(c_cap)
    assert tuple(c3.shape) == (2, 5, 4)
    with pytest.raises(RuntimeError, match="GPU device"):
        tgm.maxplus_matmul_batched_dlpack(a3.cpu(), b3.cpu())


def _assert_bits_nan(got, ref):
    """Same NaN positions, every other element bit-exact (NaN payloads may
    differ between the CPU and the GPU)."""
    got, ref = np.ascontiguousarray(got), np.ascontiguousarray(ref)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(tc.bits(got[~nan]), tc.bits(ref[~nan]))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("k", [64, 4096, 70000])
def test_backward_signed_zero_inf_nan(dtype, k):
    """dC holding -0.0, +-inf and NaN, with bins repeated inside blocks: the
    sums start from +0.0 (a bin fed only -0.0 ends +0.0), infinities of both
    signs meet (NaN), and NaN spreads to the bins it reaches, as in the
    reference's sequential sums.  Covers the LDS and the global-bin kernels."""
    from tropical_gemm import ops

    m, n = 70, 300
    rng = np.random.default_rng(k + 3)
    g = rng.standard_normal((m, n)).astype(dtype)
    am = rng.integers(0, min(k, 24), size=(m, n)).astype(np.int32)
    g[rng.random((m, n)) < 0.2] = -0.0
    g[rng.random((m, n)) < 0.01] = np.inf
    g[rng.random((m, n)) < 0.01] = -np.inf
    g[rng.random((m, n)) < 0.005] = np.nan
    am[5, :] = 3
    g[5, :] = -0.0  # a bin fed only -0.0
    print(f"[case] signed zero / inf / nan {np.dtype(dtype).name} k={k}", flush=True)
    tg_, tam = torch.from_numpy(g).to(DEV), torch.from_numpy(am).to(DEV)
    ga = ops.backward_a(tg_, tam, k).cpu().numpy()
    gb = ops.backward_b(tg_, tam, k).cpu().numpy()
    ga_ref = oracle.backward_a(g, am.astype(np.uint32), k)
    gb_ref = oracle.backward_b(g, am.astype(np.uint32), k)
    assert np.isnan(ga_ref).any() and np.isinf(ga_ref).any()
    assert tc.bits(ga_ref[5:6, 3:4])[0, 0] == 0  # +0.0
    _assert_bits_nan(ga, ga_ref)
    _assert_bits_nan(gb, gb_ref)
