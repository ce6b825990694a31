"""GPU backward (argmax scatter) and the PyTorch autograd mirror.

Gradients are accumulated with LDS atomics (a compare-and-swap of the bits
with a hardware-add fallback for f32, ds_add_f64 for f64), so the order of the
sums is not fixed.  Tolerance, per element of grad_A / grad_B:
    |gpu - oracle| <= 4 * n_terms * 2^-24 * sum(|terms|)   (f32)
    |gpu - oracle| <= 4 * n_terms * 2^-53 * sum(|terms|)   (f64)
where n_terms is how many upstream gradients land on that element; elements
with a single contribution must match exactly.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _tol_check(got, ref, g_abs_sum, n_terms, eps):
    tol = 4.0 * n_terms * eps * g_abs_sum
    diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    single = n_terms <= 1
    assert np.all(diff[single] == 0), "single-contribution elements must be exact"
    assert np.all(diff <= tol + 0.0), f"max excess {np.max(diff - tol)}"


def _contrib(argmax, g, k, which, other=None):
    """Per output element: number of terms and sum of |terms| (float64)."""
    m, n = argmax.shape
    ii, jj = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    terms = np.abs(g.astype(np.float64))
    if other is not None:
        terms = terms * np.abs(other[argmax, jj] if which == "a" else other[ii, argmax])
    shape = (m, k) if which == "a" else (k, n)
    cnt = np.zeros(shape)
    s = np.zeros(shape)
    idx = (ii, argmax) if which == "a" else (argmax, jj)
    np.add.at(cnt, idx, 1)
    np.add.at(s, idx, terms)
    return cnt, s


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
    ga_ref = oracle.backward_a(g, am, k, b if mult else None)
    gb_ref = oracle.backward_b(g, am, k, a if mult else None)
    eps = 2.0**-24 if dtype == np.float32 else 2.0**-53
    am64 = am.astype(np.int64)
    cnt, s = _contrib(am64, g, k, "a", b if mult else None)
    _tol_check(ga, ga_ref, s, cnt, eps)
    cnt, s = _contrib(am64, g, k, "b", a if mult else None)
    _tol_check(gb, gb_ref, s, cnt, eps)


# Argmax patterns that steer the f32 LDS adds down each of their paths: one
# compare-and-swap that wins (spread indices), CAS rounds that lose to other
# lanes and fall back to the hardware add (paired or clustered indices), and
# waves whose indices repeat so much that they take the hardware add outright.
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
    eps = 2.0**-24 if dtype == np.float32 else 2.0**-53
    cnt, s = _contrib(am, g, k, "a")
    _tol_check(ga, oracle.backward_a(g, am.astype(np.uint32), k), s, cnt, eps)
    cnt, s = _contrib(am, g, k, "b")
    _tol_check(gb, oracle.backward_b(g, am.astype(np.uint32), k), s, cnt, eps)


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
    np.testing.assert_allclose(ga.cpu().numpy().reshape(k, m).T, ref_a, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(gb.cpu().numpy().reshape(n, k).T, ref_b, rtol=1e-6, atol=1e-6)


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
        np.testing.assert_allclose(ga[t], oracle.backward_a(g[t], am_ref, k, b[t] if mult else None),
                                   rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(gb[t], oracle.backward_b(g[t], am_ref, k, a[t] if mult else None),
                                   rtol=1e-5, atol=1e-5)


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
    from tropical_gemm import ops, pytorch as tp

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
    _, argmax = ops.gemm(name, a.detach(), b.detach(), True)
    ga_ref, gb_ref = _scatter_reference(a, b, argmax, grad_c, name == "maxmul")
    torch.testing.assert_close(a.grad.double().cpu(), ga_ref, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(b.grad.double().cpu(), gb_ref, rtol=1e-5, atol=1e-5)


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
