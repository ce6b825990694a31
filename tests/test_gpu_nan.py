"""NaN products on every forward path: one rule, the reference CPU select rule.

The reference's argmax path keeps acc iff ``acc >= p`` (max) / ``acc <= p``
(min) for k ascending (types/max_plus.rs:66-73, min_plus.rs:66-73,
max_mul.rs:65-72).  So a NaN product replaces the running value, and the
next product replaces a NaN: the result is the first optimum after the last
NaN product, or (NaN, K-1) when the last product is NaN.  The oracle
(oracle/tg_oracle.c) restates that rule; tests/test_oracle.py pins its NaN
behaviour against those closed forms.  Here every dispatch path (named by
tg_gemm_plan, so the case provably reaches it) is compared with the oracle:
NaN at the same outputs, every other value bit-exact, argmax exact.  Value-only
calls follow the same rule (their values equal the argmax calls' values).
NaN products come from NaN operands and from infinities meeting
(+inf + -inf; 0 * inf for MaxMul).
"""
import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc
from tests.test_gpu_parity import gpu_gemm

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _plan(sr, dt, m, n, k, with_argmax, api):
    from tropical_gemm import _native

    ws = None
    if api == "min":
        es = 4 if dt in ("f32", "i32") else 8
        ws = (-(-(k * max(m, n) * es) // 256) * 256) if with_argmax else 0
    return _native.gemm_plan(sr, dt, m, n, k, with_argmax, workspace_bytes=ws)


def nan_inputs(sr, dtype, m, n, k, seed):
    """Random operands with NaN products placed at known k: the last k of
    some outputs, the middle and the start of others, infinities meeting, and
    a sprinkle of NaN operands."""
    rng = np.random.default_rng(seed)
    if sr == "maxmul":
        a = (1.0 - rng.random((m, k))).astype(dtype)
        b = (1.0 - rng.random((k, n))).astype(dtype)
    else:
        a = rng.standard_normal((m, k)).astype(dtype)
        b = rng.standard_normal((k, n)).astype(dtype)
    rows = [0, 1, 2, min(3, m - 1)]
    a[rows[0], k - 1] = np.nan          # row 0: every output's last product is NaN
    a[rows[1], k // 2] = np.nan         # row 1: a NaN in the middle resets
    a[rows[2], 0] = np.nan              # row 2: the first product is NaN
    b[k - 1, min(5, n - 1)] = np.nan    # column 5: last product NaN
    b[k // 3, min(6, n - 1)] = np.nan   # column 6
    # Infinities meeting at one k for output (4, 7) and (m-1, n-1).
    i1, j1, kk = min(4, m - 1), min(7, n - 1), k // 4
    if sr == "maxmul":
        a[i1, kk], b[kk, j1] = 0.0, np.inf
        a[m - 1, k - 2], b[k - 2, n - 1] = np.inf, 0.0
    else:
        a[i1, kk], b[kk, j1] = np.inf, -np.inf
        a[m - 1, k - 2], b[k - 2, n - 1] = -np.inf, np.inf
    # A sprinkle of NaN operands elsewhere.
    na = max(1, a.size // 2000)
    a.flat[rng.integers(0, a.size, na)] = np.nan
    b.flat[rng.integers(0, b.size, max(1, b.size // 2000))] = np.nan
    return a, b


def assert_nan_exact(c, am, c_ref, am_ref):
    nan, nan_ref = np.isnan(c), np.isnan(c_ref)
    np.testing.assert_array_equal(nan, nan_ref)
    np.testing.assert_array_equal(tc.bits(c[~nan]), tc.bits(c_ref[~nan_ref]))
    if am is not None:
        np.testing.assert_array_equal(am.astype(np.int64), am_ref.astype(np.int64))


# (semiring, dtype, m, n, k, argmax, api, expected path)
CASES = [
    ("maxplus", "f32", 67, 256, 12, True, "alloc", "shortk"),
    ("minplus", "f32", 67, 256, 12, True, "alloc", "shortk"),
    ("maxmul", "f32", 67, 256, 12, True, "alloc", "shortk"),
    ("maxplus", "f32", 67, 256, 40, False, "alloc", "shortk"),
    ("minplus", "f32", 67, 256, 40, False, "alloc", "shortk"),
    ("maxplus", "f64", 67, 256, 12, True, "alloc", "shortk"),
    ("maxplus", "f64", 67, 256, 40, False, "alloc", "shortk"),
    ("minplus", "f64", 67, 256, 40, False, "alloc", "shortk"),
    ("maxplus", "f32", 67, 45, 40, True, "alloc", "tiles_exact"),
    ("minplus", "f32", 67, 45, 40, True, "alloc", "tiles_exact"),
    ("maxmul", "f64", 67, 45, 300, True, "alloc", "tiles_exact"),
    ("maxplus", "f32", 64, 130, 512, True, "alloc", "tiles_chunked"),
    ("minplus", "f32", 64, 130, 512, True, "alloc", "tiles_chunked"),
    ("maxplus", "f32", 64, 130, 512, False, "alloc", "tiles"),
    ("maxplus", "f64", 64, 64, 640, True, "alloc", "tiles_chunked"),
    ("minplus", "f64", 64, 64, 640, True, "alloc", "tiles_chunked"),
    ("maxmul", "f64", 64, 64, 640, True, "alloc", "tiles_chunked"),
    ("maxplus", "f64", 64, 64, 640, False, "alloc", "tiles"),
    ("maxmul", "f64", 64, 64, 640, False, "alloc", "tiles"),
    ("maxplus", "f32", 256, 256, 1024, True, "ws", "dl_4x4_cl8 slices 4"),
    ("minplus", "f32", 256, 256, 1024, True, "ws", "dl_4x4_cl8 slices 4"),
    ("maxplus", "f32", 256, 256, 1024, False, "ws", "dl_4x4_cl32 split 4"),
    ("maxplus", "f32", 256, 256, 1024, True, "min", "dl_4x4_cl16"),
    ("maxmul", "f32", 256, 256, 512, True, "min", "dl_4x4_cl8"),
    ("maxplus", "f32", 512, 512, 2048, True, "min", "dl_4x4_cl16"),
    ("maxplus", "f32", 256, 256, 128, True, "alloc", "kres"),
    ("minplus", "f32", 256, 256, 128, True, "alloc", "kres"),
    ("maxmul", "f32", 256, 256, 96, True, "alloc", "kres"),
]


@pytest.mark.parametrize("sr,dt,m,n,k,argmax,api,path", CASES,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}x{c[3]}x{c[4]}-{'am' if c[5] else 'val'}-{c[6]}"
                              for c in CASES])
def test_nan_rule_per_path(sr, dt, m, n, k, argmax, api, path):
    assert _plan(sr, dt, m, n, k, argmax, api) == path
    dtype = np.float32 if dt == "f32" else np.float64
    a, b = nan_inputs(sr, dtype, m, n, k, seed=m * 7 + k)
    c, am = gpu_gemm(sr, a, b, with_argmax=argmax, api=api)
    c_ref, am_ref = oracle.gemm(sr, a, b)
    assert np.isnan(c_ref).any() and not np.isnan(c_ref).all()
    assert_nan_exact(c, am, c_ref, am_ref if argmax else None)


# The large-tile paths at full tile counts; the oracle checks the rows
# that hold NaN products plus a sample of the others (rows are independent).
BIG = [
    ("maxplus", 6144, 2048, 544, True, "dl_4x8_cl16"),
    ("minplus", 6144, 2048, 544, True, "dl_4x8_cl16"),
    ("maxplus", 4096, 4096, 96, False, "dl_8x8_cl32"),
    ("maxmul", 4096, 4096, 64, False, "dl_8x8_cl32"),
    ("maxplus", 2048, 2048, 96, False, "dl_4x8"),
    ("maxmul", 1024, 4096, 64, False, "dl_4x8"),
]


@pytest.mark.parametrize("sr,m,n,k,argmax,path", BIG,
                         ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-{c[5]}" for c in BIG])
def test_nan_rule_wide_tiles(sr, m, n, k, argmax, path):
    assert _plan(sr, "f32", m, n, k, argmax, "alloc") == path
    a, b = nan_inputs(sr, np.float32, m, n, k, seed=k)
    c, am = gpu_gemm(sr, a, b, with_argmax=argmax)
    nan_rows = np.nonzero(np.isnan(a).any(axis=1) | np.isinf(a).any(axis=1) | (a == 0).any(axis=1))[0]
    rows = np.unique(np.concatenate([nan_rows, np.arange(0, m, 257), [m - 1]]))
    c_ref, am_ref = oracle.gemm(sr, a[rows], b)
    assert_nan_exact(c[rows], am[rows] if argmax else None, c_ref, am_ref if argmax else None)
