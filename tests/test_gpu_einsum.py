"""Tropical einsum on the GPU against the brute-force oracle.

Binary contractions run one product per term, so their values and argmax are
compared bit for bit (floats included).  Longer contractions associate as the
contraction tree does; they are compared bit for bit on integer-exact data
(i32, i64, and floats holding small integers).  MaxMul is a semiring on
nonnegative values, so its data is nonnegative."""
import numpy as np
import pytest

from oracle import einsum_ref as er
from tests import tg_cases as tc

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TORCH_DT = {"f32": torch.float32, "f64": torch.float64, "i32": torch.int32, "i64": torch.int64}


def _data(rng, dt, shape, sr, small=False):
    lo = 0 if sr == "maxmul" else -9
    if dt in ("f32", "f64") and not small:
        x = rng.standard_normal(shape)
        x = np.abs(x) if sr == "maxmul" else x
    else:
        x = rng.integers(lo, 10, size=shape)
    return np.asarray(x).astype(tc.NP_DTYPES[dt])


def _dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


# (ia, ib, iy, sizes): matrix product, transposed output, several contracted
# labels, batch labels, outer products, matrix-vector, dot product, labels
# summed inside one operand, and an interleaved mix.
BINARY = [
    ("ij", "jk", "ik", dict(i=5, j=7, k=6)),
    ("ij", "jk", "ki", dict(i=5, j=7, k=6)),
    ("ijk", "jkl", "il", dict(i=4, j=3, k=5, l=6)),
    ("bij", "bjk", "bik", dict(b=3, i=4, j=5, k=6)),
    ("ibj", "jkb", "kbi", dict(b=3, i=4, j=5, k=2)),
    ("i", "j", "ij", dict(i=5, j=7)),
    ("bi", "bj", "bij", dict(b=2, i=5, j=3)),
    ("ij", "j", "i", dict(i=9, j=13)),
    ("i", "i", "", dict(i=11)),
    ("ijx", "jky", "ki", dict(i=4, j=3, k=5, x=2, y=3)),
    ("aibjc", "cjdb", "dia", dict(a=2, b=3, c=2, d=4, i=3, j=2)),
]


@pytest.mark.parametrize("dt", ["f32", "f64", "i32", "i64"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_contract_binary(sr, dt):
    from tropical_gemm import einsum as E

    rng = np.random.default_rng(300 + tc.SEMIRINGS.index(sr))
    for ia, ib, iy, size in BINARY:
        print(f"[case] contract_binary {sr} {dt} {ia},{ib}->{iy}", flush=True)
        a = _data(rng, dt, [size[x] for x in ia], sr)
        b = _data(rng, dt, [size[x] for x in ib], sr)
        y_ref, idx_ref = er.contract_binary_ref(a, b, ia, ib, iy, sr)
        y = E.contract_binary(_dev(a), _dev(b), ia, ib, iy, sr)
        np.testing.assert_array_equal(tc.bits(y.cpu().numpy()), tc.bits(y_ref))
        if idx_ref is not None:
            y2, idx = E.contract_binary(_dev(a), _dev(b), ia, ib, iy, sr, with_argmax=True)
            np.testing.assert_array_equal(tc.bits(y2.cpu().numpy()), tc.bits(y_ref))
            np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)


def test_contract_binary_ties_and_special_values():
    from tropical_gemm import einsum as E

    rng = np.random.default_rng(310)
    # Heavy ties: the first term over the contracted labels (row-major) wins.
    a = rng.integers(0, 2, size=(4, 3, 5)).astype(np.float32)
    b = rng.integers(0, 2, size=(3, 5, 6)).astype(np.float32)
    y_ref, idx_ref = er.contract_binary_ref(a, b, "ijk", "jkl", "il", "maxplus")
    y, idx = E.contract_binary(_dev(a), _dev(b), "ijk", "jkl", "il", "maxplus", with_argmax=True)
    np.testing.assert_array_equal(tc.bits(y.cpu().numpy()), tc.bits(y_ref))
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    # MinPlus distances with +inf (no edge) and rows that never beat the zero.
    a = rng.uniform(0, 100, size=(6, 4, 3)).astype(np.float32)
    b = rng.uniform(0, 100, size=(4, 3, 5)).astype(np.float32)
    a[rng.random(a.shape) < 0.3] = np.inf
    a[2] = np.inf
    y_ref, idx_ref = er.contract_binary_ref(a, b, "ijk", "jkl", "il", "minplus")
    y, idx = E.contract_binary(_dev(a), _dev(b), "ijk", "jkl", "il", "minplus", with_argmax=True)
    np.testing.assert_array_equal(tc.bits(y.cpu().numpy()), tc.bits(y_ref))
    np.testing.assert_array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    assert np.all(np.isposinf(y.cpu().numpy()[2])) and np.all(idx.cpu().numpy()[2] == 0)


# Multi-operand codes, integer-exact data.
CODES = [
    ("ij,jk,kl->il", dict(i=4, j=5, k=3, l=6)),
    ("ijk,jkl,lm->im", dict(i=3, j=4, k=2, l=5, m=3)),  # the design plan's example shape
    ("ab,bc,cd,da->", dict(a=3, b=4, c=2, d=5)),          # a ring to a scalar
    ("ab,bc,cd,da->ac", dict(a=3, b=4, c=2, d=5)),
    ("ii->i", dict(i=6)),
    ("iij,jk->ik", dict(i=4, j=5, k=3)),
    ("ij->ji", dict(i=4, j=7)),
    ("ij->", dict(i=4, j=7)),
    ("ijk->k", dict(i=3, j=4, k=5)),
    ("bij,bjk,bkl->bil", dict(b=2, i=3, j=4, k=2, l=5)),
    ("ij,ij->ij", dict(i=3, j=4)),                        # elementwise (x): batch labels only
    ("i,j,k->ijk", dict(i=2, j=3, k=4)),
]


@pytest.mark.parametrize("optimize", ["greedy", None])
@pytest.mark.parametrize("dt", ["f32", "i32", "i64"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_einsum_against_enumeration(sr, dt, optimize):
    from tropical_gemm import einsum as E

    rng = np.random.default_rng(320 + tc.SEMIRINGS.index(sr))
    for code, size in CODES:
        print(f"[case] einsum {sr} {dt} {code} optimize={optimize}", flush=True)
        ixs, iy = E.parse(code)
        ops_ = [_data(rng, dt, [size[x] for x in lab], sr, small=True) for lab in ixs]
        ref = er.einsum_ref(ixs, iy, ops_, sr)
        got = E.einsum(code, *[_dev(x) for x in ops_], semiring=sr, optimize=optimize)
        np.testing.assert_array_equal(tc.bits(np.asarray(got.cpu().numpy())), tc.bits(np.asarray(ref)))


def test_einsum_larger_network_greedy_equals_left_to_right():
    """A tensor network whose greedy order differs from left to right gives
    the same integer result."""
    from tropical_gemm import einsum as E

    rng = np.random.default_rng(330)
    code = "ab,bcd,de,ef,fca->"
    size = dict(a=6, b=40, c=5, d=30, e=3, f=7)
    ixs, iy = E.parse(code)
    path = E.einsum_path(ixs, iy, size, "greedy")
    assert path != E.einsum_path(ixs, iy, size, None)
    ops_ = [_dev(rng.integers(-50, 51, size=[size[x] for x in lab]).astype(np.int32)) for lab in ixs]
    g = E.einsum(code, *ops_, semiring="maxplus", optimize="greedy")
    s = E.einsum(code, *ops_, semiring="maxplus", optimize=None)
    assert int(g) == int(s)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_einsum_gradients(sr):
    """Gradients through the library's autograd functions: a matrix product
    written as an einsum has the GEMM's gradient, and a three-operand chain
    with a batch label matches finite differences (float64, no ties)."""
    from tropical_gemm import einsum as E
    from tropical_gemm import pytorch as tp

    rng = np.random.default_rng(340)
    lo = 0.5 if sr == "maxmul" else -1.0
    a = torch.tensor(rng.uniform(lo, 2.0, size=(5, 6)), device=DEV, requires_grad=True)
    b = torch.tensor(rng.uniform(lo, 2.0, size=(6, 4)), device=DEV, requires_grad=True)
    y = E.einsum("ij,jk->ik", a, b, semiring=sr)
    g = torch.tensor(rng.standard_normal((5, 4)), device=DEV)
    ga, gb = torch.autograd.grad(y, (a, b), g)
    fn = {"maxplus": tp.tropical_maxplus_matmul_gpu, "minplus": tp.tropical_minplus_matmul_gpu,
          "maxmul": tp.tropical_maxmul_matmul_gpu}[sr]
    y2 = fn(a, b)
    ga2, gb2 = torch.autograd.grad(y2, (a, b), g)
    assert torch.equal(y, y2)
    # The scatter sums with atomics: equal up to the order of float64 additions.
    assert torch.allclose(ga, ga2, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gb, gb2, rtol=1e-12, atol=1e-12)

    x = torch.tensor(rng.uniform(lo, 2.0, size=(2, 3, 4)), device=DEV, requires_grad=True)
    w = torch.tensor(rng.uniform(lo, 2.0, size=(2, 4, 5)), device=DEV, requires_grad=True)
    v = torch.tensor(rng.uniform(lo, 2.0, size=(5, 3)), device=DEV, requires_grad=True)
    torch.autograd.gradcheck(lambda p, q, r: E.einsum("bij,bjk,kl->bil", p, q, r, semiring=sr),
                             (x, w, v), eps=1e-6, atol=1e-5, rtol=1e-4, nondet_tol=1e-12)


def test_einsum_errors():
    from tropical_gemm import einsum as E

    a = torch.zeros((3, 4), device=DEV)
    b = torch.zeros((5, 6), device=DEV)
    with pytest.raises(ValueError, match="sizes"):
        E.einsum("ij,jk->ik", a, b)
    with pytest.raises(ValueError, match="no operand"):
        E.einsum("ij->iz", a)
    with pytest.raises(ValueError, match="dtype|float64"):
        E.einsum("ij,jk->ik", a, torch.zeros((4, 2), device=DEV, dtype=torch.float64))
    with pytest.raises(ValueError, match="semiring"):
        E.einsum("ij->i", a, semiring="plus")
    with pytest.raises(ValueError, match="device"):
        E.einsum("ij->i", torch.zeros((3, 4)))
    with pytest.raises(ValueError, match="appear in one only"):
        E.contract_binary(a, torch.zeros((4, 2), device=DEV), "ij", "jk", "k", with_argmax=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.int32, torch.int64])
@pytest.mark.parametrize("shape", [(65536, 64), (64, 65536), (1000, 37), (3, 5, 7), (65537, 2, 3),
                                   (1, 1), (4, 128, 256)])
def test_transpose_equals_torch(dtype, shape):
    """tg_transpose (the einsum's data movement) against torch's transpose,
    bit for bit: 16-byte and element kernels (aligned and ragged shapes), a
    batch beyond one grid dimension."""
    from tropical_gemm import ops

    print(f"[case] transpose {dtype} {shape}", flush=True)
    if dtype.is_floating_point:
        t = torch.randn(shape, dtype=dtype, device=DEV)
    else:
        t = torch.randint(-(1 << 30), 1 << 30, shape, dtype=dtype, device=DEV)
    got = ops.transpose(t)
    assert torch.equal(got, t.transpose(-1, -2).contiguous())


def test_einsum_operand_transposes_match_torch_copies():
    """An einsum whose operand copies are group swaps (the E1 pattern
    jik,lkj,lm->im) gives the same bits with the library's transpose as with
    torch's copies."""
    from tropical_gemm import einsum as E

    g = torch.Generator(device="cpu").manual_seed(5)
    a = torch.randn(8, 64, 16, generator=g).to(DEV)
    b = torch.randn(64, 16, 8, generator=g).to(DEV)
    c = torch.randn(64, 32, generator=g).to(DEV)
    got = E.einsum("jik,lkj,lm->im", a, b, c, semiring="maxplus")
    real = E._layout
    try:
        E._layout = lambda t, perm: t.permute(perm).contiguous()
        ref = E.einsum("jik,lkj,lm->im", a, b, c, semiring="maxplus")
    finally:
        E._layout = real
    assert torch.equal(got.contiguous().view(torch.int32), ref.contiguous().view(torch.int32))
