"""f64 direct-to-LDS kernel (tg_gemm_dl64), with and without argmax.

Large f64 problems run on it when the workspace holds the operand classes
(and B^T with argmax; tg_gemm_workspace_size); a workspace of only the B^T
minimum (argmax) or none (value-only) runs the same product on the generic
kernel.  Both must give the same bits (and argmax), equal to the oracle on
sampled rows; NaN products (NaN operands, +inf meeting -inf, 0 * inf) follow
the reference's serial rule through the class prepass and the serial rerun.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc
from tests.test_gpu_nan import nan_inputs

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _run(sr, a, b, full_ws, argmax=True):
    from tropical_gemm import _native as nat

    lib = nat.load()
    m, k = a.shape
    n = b.shape[1]
    if full_ws:
        ws_bytes = lib.tg_gemm_workspace_size(nat.DTYPE["f64"], 1, m, n, k, int(argmax))
    else:
        ws_bytes = -(-(k * max(m, n) * 8) // 256) * 256 if argmax else 0
    plan = nat.gemm_plan(sr, "f64", m, n, k, argmax, workspace_bytes=ws_bytes)
    ta = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    tb = torch.from_numpy(np.ascontiguousarray(b)).to(DEV)
    c = torch.empty(m * n, dtype=torch.float64, device=DEV)
    am = torch.empty(m * n, dtype=torch.int32, device=DEV) if argmax else None
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=DEV)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"[case] dl64 {sr} {m}x{n}x{k} argmax={argmax} {plan}", flush=True)
    nat.check(lib.tg_gemm_ws(0, nat.SEMIRING[sr], nat.DTYPE["f64"], 0, p(ta), p(tb), p(c), p(am),
                             m, n, k, p(ws), ws_bytes, stream))
    torch.cuda.synchronize()
    return (plan, c.cpu().numpy().reshape(m, n),
            am.cpu().numpy().reshape(m, n) if argmax else None)


def _check(c, am, c_ref, am_ref):
    nan = np.isnan(c_ref)
    np.testing.assert_array_equal(np.isnan(c), nan)
    np.testing.assert_array_equal(tc.bits(c[~nan]), tc.bits(c_ref[~nan]))
    np.testing.assert_array_equal(am.astype(np.int64), am_ref.astype(np.int64))


def _operands(sr, m, n, k, seed):
    rng = np.random.default_rng(seed)
    if sr == "maxmul":
        a = 1.0 - rng.random((m, k))
        b = 1.0 - rng.random((k, n))
        a = np.round(a * 8) / 8 + 1 / 16  # ties, no zeros
        b = np.round(b * 8) / 8 + 1 / 16
    else:
        a = np.round(rng.standard_normal((m, k)) * 4) / 4  # ties across k and chunks
        b = np.round(rng.standard_normal((k, n)) * 4) / 4
    return a, b


@pytest.mark.parametrize("sr", ["maxplus", "minplus", "maxmul"])
@pytest.mark.parametrize("m,n,k", [(1024, 4096, 640), (1000, 4092, 672)])
def test_dl64_matches_generic_and_oracle(sr, m, n, k):
    a, b = _operands(sr, m, n, k, seed=m + k)
    plan, c, am = _run(sr, a, b, full_ws=True)
    assert plan == "dl64_4x8_cl16"
    plan0, c0, am0 = _run(sr, a, b, full_ws=False)
    assert plan0 == "tiles_chunked"
    _check(c, am, c0, am0)
    rows = np.array([0, 1, 63, 64, 500, m - 1])
    c_ref, am_ref = oracle.gemm(sr, a[rows], b)
    _check(c[rows], am[rows], c_ref, am_ref)


@pytest.mark.parametrize("sr", ["maxplus", "minplus", "maxmul"])
def test_dl64_nan_rule(sr):
    m, n, k = 1024, 4096, 640
    a, b = nan_inputs(sr, np.float64, m, n, k, seed=17)
    plan, c, am = _run(sr, a, b, full_ws=True)
    assert plan == "dl64_4x8_cl16"
    special = ~np.isfinite(a).all(axis=1) | (a == 0).any(axis=1)
    rows = np.unique(np.concatenate([np.nonzero(special)[0], np.arange(0, m, 97), [m - 1]]))
    c_ref, am_ref = oracle.gemm(sr, a[rows], b)
    assert np.isnan(c_ref).any()
    _check(c[rows], am[rows], c_ref, am_ref)


def _check_values(c, c_ref):
    nan = np.isnan(c_ref)
    np.testing.assert_array_equal(np.isnan(c), nan)
    np.testing.assert_array_equal(tc.bits(c[~nan]), tc.bits(c_ref[~nan]))


@pytest.mark.parametrize("sr", ["maxplus", "minplus", "maxmul"])
@pytest.mark.parametrize("m,n,k", [(1024, 4096, 640), (1000, 4092, 672)])
def test_dl64_value_only_matches_generic_and_oracle(sr, m, n, k):
    """Value-only on the f64 direct-to-LDS kernel: the same bits as the
    generic kernel (run by the same call without a workspace) and the
    oracle's values on sampled rows.  The data has no zeros, so no +-0 tie
    makes the sign of a value-only maximum open."""
    a, b = _operands(sr, m, n, k, seed=3 * m + k)
    if sr != "maxmul":
        a[a == 0] = 0.125
        b[b == 0] = -0.125
    plan, c, _ = _run(sr, a, b, full_ws=True, argmax=False)
    assert plan == "dl64_4x8"
    plan0, c0, _ = _run(sr, a, b, full_ws=False, argmax=False)
    assert plan0 == "tiles"
    _check_values(c, c0)
    rows = np.array([0, 1, 63, 64, 500, m - 1])
    c_ref, _ = oracle.gemm(sr, a[rows], b)
    _check_values(c[rows], c_ref)


@pytest.mark.parametrize("sr", ["maxplus", "minplus", "maxmul"])
def test_dl64_value_only_nan_rule(sr):
    m, n, k = 1024, 4096, 640
    a, b = nan_inputs(sr, np.float64, m, n, k, seed=23)
    plan, c, _ = _run(sr, a, b, full_ws=True, argmax=False)
    assert plan == "dl64_4x8"
    special = ~np.isfinite(a).all(axis=1) | (a == 0).any(axis=1)
    rows = np.unique(np.concatenate([np.nonzero(special)[0], np.arange(0, m, 97), [m - 1]]))
    c_ref, _ = oracle.gemm(sr, a[rows], b)
    assert np.isnan(c_ref).any()
    _check_values(c[rows], c_ref)


@pytest.mark.parametrize("argmax", [True, False])
@pytest.mark.parametrize("sr", ["maxplus", "minplus"])
def test_dl64_column_major(sr, argmax):
    """Column-major calls run the row-major product C^T = B^T (x) A^T on the
    same kernel (here M' = 4096, N' = 1024)."""
    from tests.test_gpu_parity import gpu_gemm
    from tropical_gemm import _native as nat

    m, n, k = 1024, 4096, 640
    plan = nat.gemm_plan(sr, "f64", m, n, k, argmax, layout="col")
    assert plan == ("dl64_4x8_cl16" if argmax else "dl64_4x8")
    a, b = _operands(sr, m, n, k, seed=91)
    a[a == 0] = 0.125
    b[b == 0] = -0.125
    print(f"[case] dl64 col-major {sr} argmax={argmax}", flush=True)
    c, am = gpu_gemm(sr, a, b, with_argmax=argmax, layout="col")
    rows = np.array([0, 5, 511, m - 1])
    c_ref, am_ref = oracle.gemm(sr, a[rows], b)
    _check_values(c[rows], c_ref)
    if argmax:
        np.testing.assert_array_equal(am[rows].astype(np.int64), am_ref.astype(np.int64))


@pytest.mark.parametrize("argmax", [True, False])
def test_dl64_strided_batched(argmax):
    """Two batch items, each with its own operand classes (a NaN in item 1
    only) and, with argmax, its own B^T."""
    from tropical_gemm import _native as nat, ops

    batch, m, n, k = 2, 512, 4096, 640
    plan = nat.gemm_plan("maxplus", "f64", m, n, k, argmax, batch=batch,
                         strides=(m * k, k * n, m * n))
    assert plan == ("dl64_4x8_cl16" if argmax else "dl64_4x8")
    rng = np.random.default_rng(92)
    a = np.round(rng.standard_normal((batch, m, k)) * 4) / 4
    b = np.round(rng.standard_normal((batch, k, n)) * 4) / 4
    a[a == 0] = 0.125
    b[b == 0] = -0.125
    a[1, 3, k // 2] = np.nan
    print(f"[case] dl64 batched argmax={argmax}", flush=True)
    c, am = ops.gemm_batched("maxplus", torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV),
                             argmax)
    torch.cuda.synchronize()
    c = c.cpu().numpy()
    am = am.cpu().numpy() if argmax else None
    rows = np.array([0, 3, 64, m - 1])
    for z in range(batch):
        c_ref, am_ref = oracle.gemm("maxplus", a[z][rows], b[z])
        _check_values(c[z][rows], c_ref)
        if argmax:
            np.testing.assert_array_equal(am[z][rows].astype(np.int64), am_ref.astype(np.int64))
