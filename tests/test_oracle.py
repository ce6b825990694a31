"""Pins the CPU oracle (oracle/tg_oracle.c) before anything is checked against it.

* every golden fixture the reference ships (values bit-exact, argmax exact);
* the reference's hand-computed cases (tie rule, -inf identity, K = 0);
* an independent brute-force numpy formulation on random small shapes for
  all dtypes and semirings, including heavy ties and integer wrap-around;
* the backward loops against closed forms and np.add.at;
* the single-thread baseline restatement against the oracle.
"""
import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc


@pytest.mark.parametrize("path", tc.fixture_paths(), ids=lambda p: p.split("fixtures/")[-1])
def test_oracle_matches_golden_fixture(path):
    fx = tc.load_fixture(path)
    if fx["a"].ndim == 3:
        c, am = oracle.gemm_batched(fx["algebra"], fx["a"], fx["b"])
    else:
        c, am = oracle.gemm(fx["algebra"], fx["a"], fx["b"])
    np.testing.assert_array_equal(tc.bits(c), tc.bits(fx["c"]))
    np.testing.assert_array_equal(am.astype(np.int64), fx["argmax"])


def test_fixture_inventory():
    # 3 algebras x 2 float dtypes x (5 shapes + 2 batched) + 6 special cases.
    assert len(tc.fixture_paths()) == 48


@pytest.mark.parametrize("case", tc.HAND_CASES, ids=lambda c: c[5])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_oracle_hand_cases(case, dtype):
    sr, a, b, c_exp, am_exp, _src = case
    c, am = oracle.gemm(sr, a.astype(dtype), b.astype(dtype))
    np.testing.assert_array_equal(c, np.array(c_exp, dtype=dtype))
    np.testing.assert_array_equal(am, np.array(am_exp))


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_oracle_integer_hand_cases(dtype):
    # tropical-gemm/src/api.rs:918-957 (i32/i64 MaxPlus and MinPlus).
    a = np.arange(1, 7, dtype=dtype).reshape(2, 3)
    b = np.arange(1, 7, dtype=dtype).reshape(3, 2)
    c, _ = oracle.gemm("maxplus", a, b)
    np.testing.assert_array_equal(c, [[8, 9], [11, 12]])
    c, _ = oracle.gemm("minplus", a, b)
    np.testing.assert_array_equal(c, [[2, 3], [5, 6]])


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
@pytest.mark.parametrize("dt", ["f32", "f64", "i32", "i64"])
def test_oracle_matches_brute_force(sr, dt):
    rng = np.random.default_rng(1234 + hash((sr, dt)) % 1000)
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in [(1, 1, 1), (3, 5, 7), (17, 33, 9), (40, 70, 31)]:
        a = tc.rng_matrix(rng, dtype, (m, k), -20, 20)
        b = tc.rng_matrix(rng, dtype, (k, n), -20, 20)
        c, am = oracle.gemm(sr, a, b)
        c_bf, am_bf = tc.brute_force(sr, a, b)
        np.testing.assert_array_equal(tc.bits(c), tc.bits(c_bf))
        np.testing.assert_array_equal(am.astype(np.int64), am_bf)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_oracle_ties_first_k(sr):
    # Few distinct values -> most outputs have several maximisers.
    rng = np.random.default_rng(7)
    a = rng.integers(0, 3, size=(23, 41)).astype(np.float32)
    b = rng.integers(0, 3, size=(41, 19)).astype(np.float32)
    c, am = oracle.gemm(sr, a, b)
    c_bf, am_bf = tc.brute_force(sr, a, b)
    np.testing.assert_array_equal(c, c_bf)
    np.testing.assert_array_equal(am.astype(np.int64), am_bf)


def test_oracle_integer_wraps():
    # Release-build Rust `+` wraps (types/scalar.rs:94-102).
    a = np.array([[2**31 - 1, 5]], dtype=np.int32)
    b = np.array([[1], [2]], dtype=np.int32)
    c, am = oracle.gemm("maxplus", a, b)
    # 2^31-1 + 1 wraps to -2^31, so k = 1 (5 + 2 = 7) wins.
    assert c[0, 0] == 7 and am[0, 0] == 1
    c, am = oracle.gemm("minplus", a, b)
    assert c[0, 0] == -(2**31) and am[0, 0] == 0


def test_oracle_k_zero_gives_tropical_zero():
    for sr, z in [("maxplus", -np.inf), ("minplus", np.inf), ("maxmul", 0.0)]:
        c, am = oracle.gemm(sr, np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32))
        assert np.all(c == z) and np.all(am == 0)


def test_oracle_special_values():
    # MinPlus with +inf entries (test_tropical_gemm.py:529-538): inf never wins.
    a = np.array([[np.inf, 1.0], [2.0, np.inf]], dtype=np.float32)
    b = np.array([[1.0, np.inf], [np.inf, 3.0]], dtype=np.float32)
    c, am = oracle.gemm("minplus", a, b)
    np.testing.assert_array_equal(c, [[np.inf, 4.0], [3.0, np.inf]])
    np.testing.assert_array_equal(am, [[0, 1], [0, 0]])
    # MaxMul with zeros (test_tropical_gemm.py:541-554): all products <= 0 keep (0, 0).
    a = np.array([[0.0, -1.0]], dtype=np.float32)
    b = np.array([[5.0], [2.0]], dtype=np.float32)
    c, am = oracle.gemm("maxmul", a, b)
    assert c[0, 0] == 0.0 and am[0, 0] == 0


def test_oracle_signed_zero_first_occurrence():
    # Select rule keeps the earlier of equal values: -0 then +0 stays -0.
    a = np.array([[-0.0, 0.0]], dtype=np.float32)
    b = np.array([[-0.0], [0.0]], dtype=np.float32)
    c, am = oracle.gemm("maxplus", a, b)
    assert np.signbit(c[0, 0]) and am[0, 0] == 0


def _backward_ref(grad_c, argmax, k, other=None, which="a"):
    m, n = grad_c.shape
    out = np.zeros((m, k) if which == "a" else (k, n), dtype=np.float64)
    ii, jj = np.meshgrid(np.arange(m), np.arange(n), indexing="ij")
    g = grad_c.astype(np.float64)
    if other is not None:
        g = g * (other[argmax, jj] if which == "a" else other[ii, argmax])
    if which == "a":
        np.add.at(out, (ii, argmax), g)
    else:
        np.add.at(out, (argmax, jj), g)
    return out


def test_oracle_backward_closed_forms():
    # tropical-gemm/src/api.rs:1211-1260: all argmax = 2, grad_c = 1.
    a = np.arange(1, 7, dtype=np.float64).reshape(2, 3)
    b = np.arange(1, 7, dtype=np.float64).reshape(3, 2)
    _, am = oracle.gemm("maxplus", a, b)
    g = np.ones((2, 2))
    ga = oracle.backward_a(g, am, 3)
    gb = oracle.backward_b(g, am, 3)
    np.testing.assert_array_equal(ga, [[0, 0, 2], [0, 0, 2]])
    np.testing.assert_array_equal(gb, [[0, 0], [0, 0], [2, 2]])


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("mult", [False, True])
def test_oracle_backward_matches_add_at(dtype, mult):
    rng = np.random.default_rng(5)
    m, k, n = 37, 23, 29
    a = rng.standard_normal((m, k)).astype(dtype)
    b = rng.standard_normal((k, n)).astype(dtype)
    _, am = oracle.gemm("maxmul" if mult else "maxplus", a, b)
    g = rng.standard_normal((m, n)).astype(dtype)
    ga = oracle.backward_a(g, am, k, b if mult else None)
    gb = oracle.backward_b(g, am, k, a if mult else None)
    tol = 1e-5 if dtype == np.float32 else 1e-12
    np.testing.assert_allclose(ga, _backward_ref(g, am.astype(np.int64), k, b if mult else None, "a"),
                               rtol=tol, atol=tol)
    np.testing.assert_allclose(gb, _backward_ref(g, am.astype(np.int64), k, a if mult else None, "b"),
                               rtol=tol, atol=tol)
    if not mult:
        # Invariant: every upstream gradient lands exactly once (api.rs:1295-1298).
        assert abs(ga.sum(dtype=np.float64) - g.sum(dtype=np.float64)) < 1e-3
        assert abs(gb.sum(dtype=np.float64) - g.sum(dtype=np.float64)) < 1e-3


def test_oracle_backward_skips_out_of_range_index():
    g = np.ones((1, 2), np.float32)
    am = np.array([[0, 7]], dtype=np.uint32)  # 7 >= k: skipped (api.rs:575-582)
    ga = oracle.backward_a(g, am, 3)
    np.testing.assert_array_equal(ga, [[1, 0, 0]])


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_portable_baseline_equals_oracle(sr):
    rng = np.random.default_rng(11)
    a = rng.standard_normal((67, 301)).astype(np.float32)
    b = rng.standard_normal((301, 130)).astype(np.float32)
    c1, a1 = oracle.gemm(sr, a, b)
    c2, a2 = oracle.portable_argmax_f32(sr, a, b)
    np.testing.assert_array_equal(tc.bits(c1), tc.bits(c2))
    np.testing.assert_array_equal(a1, a2)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_portable_baseline_f64_equals_oracle(sr):
    # Ties from a coarse grid; K = 300 crosses the 256-k block.
    rng = np.random.default_rng(13)
    a = np.round(rng.standard_normal((67, 300)) * 4) / 4
    b = np.round(rng.standard_normal((300, 130)) * 4) / 4
    if sr == "maxmul":
        a, b = np.abs(a), np.abs(b)
    c1, a1 = oracle.gemm(sr, a, b)
    c2, a2 = oracle.portable_argmax(sr, a, b)
    np.testing.assert_array_equal(tc.bits(c1), tc.bits(c2))
    np.testing.assert_array_equal(a1, a2)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_portable_baseline_i32_equals_oracle(sr):
    # K = 300 crosses the 256-k block (the argmax carries k_offset); ties,
    # and wrapping sums near the int32 limits.
    rng = np.random.default_rng(12)
    for lo, hi in ((-1000, 1001), (0, 3), (2**31 - 60, 2**31 - 1)):
        a = rng.integers(lo, hi, size=(67, 300)).astype(np.int32)
        b = rng.integers(-5, 60, size=(300, 130)).astype(np.int32)
        c1, a1 = oracle.gemm(sr, a, b)
        c2, a2 = oracle.portable_argmax(sr, a, b)
        np.testing.assert_array_equal(c1, c2)
        np.testing.assert_array_equal(a1, a2)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_portable_baselines_i64_equal_oracle(sr):
    # The i64 argmax and value-only restatements: K = 300 crosses the 256-k
    # block, 67 x 130 leaves partial 4 x 4 micro-blocks; ties, and wrapping
    # sums and products near the int64 limits.  The value path is also
    # pinned by numpy brute force on a corner (wrapping adds and products).
    rng = np.random.default_rng(15)
    for lo, hi in ((-10**12, 10**12), (0, 3), (2**63 - 60, 2**63 - 1)):
        a = rng.integers(lo, hi, size=(67, 300), dtype=np.int64)
        b = rng.integers(-5, 60, size=(300, 130)).astype(np.int64)
        c1, a1 = oracle.gemm(sr, a, b)
        c2, a2 = oracle.portable_argmax(sr, a, b)
        np.testing.assert_array_equal(c1, c2)
        np.testing.assert_array_equal(a1, a2)
        c3 = oracle.portable_gemm(sr, a, b)
        np.testing.assert_array_equal(c1, c3)
        with np.errstate(over="ignore"):
            prod = (a[:5, :, None] * b[None, :, :7]) if sr == "maxmul" else (a[:5, :, None] + b[None, :, :7])
        ref = prod.min(axis=1) if sr == "minplus" else prod.max(axis=1)
        np.testing.assert_array_equal(c3[:5, :7], ref)
    # int32 value path against the oracle; empty K gives the tropical zero.
    a = rng.integers(-1000, 1001, size=(67, 300)).astype(np.int32)
    b = rng.integers(-1000, 1001, size=(300, 130)).astype(np.int32)
    np.testing.assert_array_equal(oracle.portable_gemm(sr, a, b),
                                  oracle.gemm(sr, a, b, with_argmax=False)[0])
    z = oracle.portable_gemm(sr, np.zeros((3, 0), np.int64), np.zeros((0, 5), np.int64))
    zero = {"maxplus": np.iinfo(np.int64).min, "minplus": np.iinfo(np.int64).max, "maxmul": 0}[sr]
    np.testing.assert_array_equal(z, np.full((3, 5), zero, np.int64))


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_avx2_value_baseline_equals_oracle(sr):
    # 300 x 600 x 270 crosses every block edge of the 256/256/512 tiling and
    # leaves partial 8 x 8 micro-blocks; MaxMul on positive data.
    rng = np.random.default_rng(13)
    if sr == "maxmul":
        a = (1.0 - rng.random((300, 600))).astype(np.float32)
        b = (1.0 - rng.random((600, 270))).astype(np.float32)
    else:
        a = rng.standard_normal((300, 600)).astype(np.float32)
        b = rng.standard_normal((600, 270)).astype(np.float32)
    c1, _ = oracle.gemm(sr, a, b, with_argmax=False)
    c2 = oracle.avx2_gemm_f32(sr, a, b)
    np.testing.assert_array_equal(tc.bits(c1), tc.bits(c2))
    # Empty K: the tropical zero everywhere.
    z = oracle.avx2_gemm_f32(sr, np.zeros((3, 0), np.float32), np.zeros((0, 5), np.float32))
    np.testing.assert_array_equal(z, np.full((3, 5), {"maxplus": -np.inf, "minplus": np.inf,
                                                      "maxmul": 0.0}[sr], np.float32))


def test_avx2_maxplus_f64_baseline_equals_oracle():
    # 300 x 600 x 270 crosses every block edge of the 128/128/256 tiling and
    # leaves partial 4 x 4 micro-blocks; values with ties across k (quarters).
    rng = np.random.default_rng(14)
    a = np.round(rng.standard_normal((300, 600)) * 4) / 4
    b = np.round(rng.standard_normal((600, 270)) * 4) / 4
    c1, _ = oracle.gemm("maxplus", a, b, with_argmax=False)
    c2 = oracle.avx2_gemm_maxplus_f64("maxplus", a, b)
    np.testing.assert_array_equal(tc.bits(c1), tc.bits(c2))
    # Brute force on a corner: max over k of a[i, k] + b[k, j].
    np.testing.assert_array_equal(c2[:5, :7], (a[:5, :, None] + b[None, :, :7]).max(axis=1))
    z = oracle.avx2_gemm_maxplus_f64("maxplus", np.zeros((3, 0)), np.zeros((0, 5)))
    np.testing.assert_array_equal(z, np.full((3, 5), -np.inf))
    with pytest.raises(ValueError):
        oracle.avx2_gemm_maxplus_f64("minplus", a, b)


@pytest.mark.parametrize("sr", ["maxplus", "minplus", "maxmul"])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_oracle_nan_closed_forms(sr, dtype):
    """NaN products under the reference's keep-rule (acc >= p for max,
    acc <= p for min): a NaN product replaces the running value and the next
    product replaces the NaN, so a row's result is the first optimum of the
    products after its last NaN product, or (NaN, that k) when the NaN comes
    last; rows whose last product is NaN end NaN, and a product that only
    ties the pre-NaN optimum after the reset still wins (no memory survives
    the NaN).  Checked one output per row, k = 0..5, with A[i, k] the product
    itself (B = the semiring's one), against the closed form, not the loop."""
    one = 1.0 if sr == "maxmul" else 0.0
    nan = np.nan
    rows = [
        [1, nan, 3, 2, 3, 0],    # reset at 1, then first optimum of [3, 2, 3, 0]
        [5, 4, 3, 2, 1, nan],    # NaN last: (NaN, 5)
        [nan, 2, 2, 1, 0, 2],    # NaN first: first optimum of the rest
        [9, 1, nan, 1, 0, 0.5],  # the pre-NaN 9 is forgotten
        [nan, nan, nan, nan, nan, 7],
        [2, 2, 2, 2, 2, 2],      # no NaN: first optimum, k = 0
    ]
    if sr == "maxmul":
        rows = [[abs(x) if x == x else x for x in r] for r in rows]
    a = np.array(rows, dtype=dtype)
    b = np.full((a.shape[1], 1), one, dtype=dtype)
    c, am = oracle.gemm(sr, a, b)
    better = (lambda x, y: x < y) if sr == "minplus" else (lambda x, y: x > y)
    for i, r in enumerate(rows):
        last_nan = max([k for k, x in enumerate(r) if x != x], default=-1)
        if last_nan == len(r) - 1:
            assert np.isnan(c[i, 0]) and am[i, 0] == last_nan
            continue
        tail = list(range(last_nan + 1, len(r)))
        best = tail[0]
        for k in tail[1:]:
            if better(r[k], r[best]):
                best = k
        assert c[i, 0] == dtype(r[best]) and am[i, 0] == best, (i, c[i, 0], am[i, 0], best)


def test_oracle_nan_from_infinities():
    """-inf + inf and 0 * inf are NaN products: the same reset."""
    a = np.array([[3.0, -np.inf, 1.0, 0.5]], dtype=np.float32)
    b = np.array([[0.0], [np.inf], [0.0], [0.0]], dtype=np.float32)
    c, am = oracle.gemm("maxplus", a, b)
    assert c[0, 0] == 1.0 and am[0, 0] == 2          # 3 forgotten after the NaN at k = 1
    a = np.array([[0.5, 0.0, 0.25, 0.125]], dtype=np.float32)
    b = np.array([[1.0], [np.inf], [1.0], [1.0]], dtype=np.float32)
    c, am = oracle.gemm("maxmul", a, b)
    assert c[0, 0] == 0.25 and am[0, 0] == 2
