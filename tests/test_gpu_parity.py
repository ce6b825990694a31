"""GPU parity: every forward entry point of the C ABI against the oracle,
bit-exact (values compared as bit patterns, argmax exactly)."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TORCH_DT = {np.dtype(np.float32): torch.float32, np.dtype(np.float64): torch.float64,
            np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64}
DT_NAME = {np.dtype(np.float32): "f32", np.dtype(np.float64): "f64",
           np.dtype(np.int32): "i32", np.dtype(np.int64): "i64"}


def _nat():
    from tropical_gemm import _native

    return _native


def _dev(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def min_workspace(a, k, m, n, with_argmax):
    """The documented minimum workspace: k x max(m, n) elements per product
    for argmax calls (B^T staging), rounded up to 256 bytes."""
    if not with_argmax:
        return 0
    return -(-(k * max(m, n) * a.dtype.itemsize) // 256) * 256


def gpu_gemm(sr, a, b, with_argmax=True, layout="row", api="alloc"):
    """Run tg_gemm (api='alloc') or tg_gemm_ws through ctypes, with
    tg_gemm_workspace_size bytes (api='ws') or the documented minimum
    (api='min', which runs products that need more than the minimum on the
    kernels that do not).  For layout='col' the numpy inputs are row-major
    logical matrices that are handed over in column-major storage; results
    come back row-major."""
    nat = _nat()
    lib = nat.load()
    m, k = a.shape
    n = b.shape[1]
    if layout == "col":
        ta, tb = _dev(np.asfortranarray(a).T.copy()), _dev(np.asfortranarray(b).T.copy())
    else:
        ta, tb = _dev(a), _dev(b)
    c = torch.empty(m * n, dtype=TORCH_DT[a.dtype], device=DEV)
    am = torch.empty(m * n, dtype=torch.int32, device=DEV) if with_argmax else None
    dt = nat.DTYPE[DT_NAME[a.dtype]]
    lay = nat.LAYOUT[layout]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if api == "alloc":
        nat.check(lib.tg_gemm(0, nat.SEMIRING[sr], dt, lay, _p(ta), _p(tb), _p(c), _p(am), m, n, k,
                              stream))
    else:
        if api == "min":
            ws_bytes = min_workspace(a, k, m, n, with_argmax)
        else:
            ws_bytes = lib.tg_gemm_workspace_size(dt, 1, m, n, k, int(with_argmax))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
        nat.check(lib.tg_gemm_ws(0, nat.SEMIRING[sr], dt, lay, _p(ta), _p(tb), _p(c), _p(am), m,
                                 n, k, _p(ws), ws_bytes, stream))
    torch.cuda.synchronize()
    if layout == "col":
        c_np = c.cpu().numpy().reshape(n, m).T
        am_np = am.cpu().numpy().reshape(n, m).T if with_argmax else None
    else:
        c_np = c.cpu().numpy().reshape(m, n)
        am_np = am.cpu().numpy().reshape(m, n) if with_argmax else None
    return c_np, am_np


def assert_exact(c, am, c_ref, am_ref):
    np.testing.assert_array_equal(tc.bits(c), tc.bits(c_ref))
    if am is not None:
        np.testing.assert_array_equal(am.astype(np.int64), am_ref.astype(np.int64))


# ---------------------------------------------------------------------------
# Golden fixtures through the C ABI (2-D via tg_gemm, 3-D via strided batched)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("path", tc.fixture_paths(), ids=lambda p: p.split("fixtures/")[-1])
def test_golden_fixture_on_gpu(path):
    from tropical_gemm import ops

    fx = tc.load_fixture(path)
    if fx["a"].ndim == 3:
        c, am = ops.gemm_batched(fx["algebra"], _dev(fx["a"]), _dev(fx["b"]), True)
    else:
        c, am = ops.gemm(fx["algebra"], _dev(fx["a"]), _dev(fx["b"]), True)
    assert_exact(c.cpu().numpy(), am.cpu().numpy(), fx["c"], fx["argmax"])


@pytest.mark.parametrize("case", tc.HAND_CASES, ids=lambda c: c[5])
def test_hand_cases_on_gpu(case):
    sr, a, b, c_exp, am_exp, _ = case
    for dtype in (np.float32, np.float64):
        c, am = gpu_gemm(sr, a.astype(dtype), b.astype(dtype))
        np.testing.assert_array_equal(c, np.array(c_exp, dtype=dtype))
        np.testing.assert_array_equal(am, np.array(am_exp))


# ---------------------------------------------------------------------------
# Random shapes: every dtype x semiring x {value, argmax}, ragged edges
# ---------------------------------------------------------------------------

SHAPES = [(1, 1, 1), (1, 37, 1), (5, 3, 7), (64, 32, 64), (129, 65, 63), (130, 31, 200),
          (257, 100, 129), (33, 1000, 17)]


@pytest.mark.parametrize("dt", ["f32", "f64", "i32", "i64"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_random_shapes_argmax(sr, dt):
    rng = np.random.default_rng(100 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in SHAPES:
        print(f"[case] argmax {sr} {dt} m={m} k={k} n={n}", flush=True)
        a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        c, am = gpu_gemm(sr, a, b, True)
        c_ref, am_ref = oracle.gemm(sr, a, b)
        assert_exact(c, am, c_ref, am_ref)


@pytest.mark.parametrize("dt", ["f32", "f64", "i32", "i64"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_random_shapes_value_only(sr, dt):
    rng = np.random.default_rng(200 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in SHAPES:
        a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        c, _ = gpu_gemm(sr, a, b, False)
        c_ref, _ = oracle.gemm(sr, a, b, with_argmax=False)
        assert_exact(c, None, c_ref, None)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_column_major_layout(sr):
    rng = np.random.default_rng(9)
    for dtype in (np.float32, np.int64):
        a = tc.rng_matrix(rng, dtype, (45, 77), -50, 50)
        b = tc.rng_matrix(rng, dtype, (77, 29), -50, 50)
        c_ref, am_ref = oracle.gemm(sr, a, b)
        for api in ("alloc", "ws"):
            c, am = gpu_gemm(sr, a, b, True, layout="col", api=api)
            assert_exact(c, am, c_ref, am_ref)
            c, _ = gpu_gemm(sr, a, b, False, layout="col", api=api)
            assert_exact(c, None, c_ref, None)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
@pytest.mark.parametrize("dt", ["f32", "i32"])
def test_heavy_ties_first_k(sr, dt):
    # Values in {0,1,2}: most outputs have many maximisers spread over chunks.
    rng = np.random.default_rng(77)
    dtype = tc.NP_DTYPES[dt]
    a = rng.integers(0, 3, size=(150, 333)).astype(dtype)
    b = rng.integers(0, 3, size=(333, 70)).astype(dtype)
    c, am = gpu_gemm(sr, a, b)
    c_ref, am_ref = oracle.gemm(sr, a, b)
    assert_exact(c, am, c_ref, am_ref)


def test_integer_wraparound_matches_cpu_semantics():
    rng = np.random.default_rng(3)
    for dtype in (np.int32, np.int64):
        info = np.iinfo(dtype)
        a = rng.integers(info.max - 50, info.max, size=(70, 90), dtype=dtype)
        b = rng.integers(-5, 60, size=(90, 40)).astype(dtype)
        for sr in tc.SEMIRINGS:
            c, am = gpu_gemm(sr, a, b)
            c_ref, am_ref = oracle.gemm(sr, a, b)
            assert_exact(c, am, c_ref, am_ref)


def test_special_values():
    rng = np.random.default_rng(4)
    a = rng.standard_normal((80, 96)).astype(np.float32)
    b = rng.standard_normal((96, 72)).astype(np.float32)
    a[rng.random(a.shape) < 0.2] = np.inf
    b[rng.random(b.shape) < 0.2] = np.inf
    c, am = gpu_gemm("minplus", a, b)
    assert_exact(c, am, *oracle.gemm("minplus", a, b))
    a2 = np.where(np.isinf(a), -np.inf, a).astype(np.float32)
    b2 = np.where(np.isinf(b), -np.inf, b).astype(np.float32)
    c, am = gpu_gemm("maxplus", a2, b2)
    assert_exact(c, am, *oracle.gemm("maxplus", a2, b2))
    # all-(-inf) rows: C = -inf, argmax 0
    a2[3, :] = -np.inf
    c, am = gpu_gemm("maxplus", a2, b2)
    assert np.all(np.isneginf(c[3])) and np.all(am[3] == 0)
    # MaxMul with zeros and negatives: products <= 0 never beat the zero.
    a3 = rng.integers(-2, 3, size=(64, 50)).astype(np.float32)
    b3 = rng.integers(-2, 3, size=(50, 64)).astype(np.float32)
    c, am = gpu_gemm("maxmul", a3, b3)
    assert_exact(c, am, *oracle.gemm("maxmul", a3, b3))


def test_signed_zero_first_occurrence():
    # -0 (k=0) and +0 (k=1..) tie at the maximum: the CPU keeps -0 / index 0.
    a = np.zeros((4, 70), np.float32)
    a[:, 0] = -0.0
    b = np.zeros((70, 5), np.float32)
    b[0, :] = -0.0
    b[1:, :] = -1.0
    b[40, :] = 0.0
    c, am = gpu_gemm("maxplus", a, b)
    c_ref, am_ref = oracle.gemm("maxplus", a, b)
    assert_exact(c, am, c_ref, am_ref)
    assert np.all(np.signbit(c)) and np.all(am == 0)


def test_k_zero_and_empty():
    for sr, z in [("maxplus", -np.inf), ("minplus", np.inf), ("maxmul", 0.0)]:
        c, am = gpu_gemm(sr, np.zeros((5, 0), np.float32), np.zeros((0, 3), np.float32))
        assert np.all(c == z) and np.all(am == 0)
    c, am = gpu_gemm("maxplus", np.zeros((0, 4), np.float32), np.zeros((4, 3), np.float32))
    assert c.shape == (0, 3)


def test_unaligned_and_odd_strides_use_scalar_path():
    # K, N not multiples of 4 -> scalar tile loads; offset pointers -> unaligned.
    from tropical_gemm import _native as nat

    lib = nat.load()
    rng = np.random.default_rng(8)
    m, k, n = 70, 45, 53
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    ta = _dev(np.concatenate([[0.0], a.ravel()]).astype(np.float32))
    tb = _dev(np.concatenate([[0.0], b.ravel()]).astype(np.float32))
    c = torch.empty(m * n, dtype=torch.float32, device=DEV)
    am = torch.empty(m * n, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm(0, 0, 0, 0, ctypes.c_void_p(ta.data_ptr() + 4),
                          ctypes.c_void_p(tb.data_ptr() + 4), _p(c), _p(am), m, n, k, None))
    torch.cuda.synchronize()
    assert_exact(c.cpu().numpy().reshape(m, n), am.cpu().numpy().reshape(m, n),
                 *oracle.gemm("maxplus", a, b))


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_strided_batched_with_gaps(sr):
    from tropical_gemm import _native as nat

    lib = nat.load()
    rng = np.random.default_rng(12)
    batch, m, k, n = 3, 33, 70, 41
    sa, sb, sc = m * k + 5, k * n + 3, m * n + 7
    a = rng.standard_normal(batch * sa).astype(np.float32)
    b = rng.standard_normal(batch * sb).astype(np.float32)
    ta, tb = _dev(a), _dev(b)
    c = torch.zeros(batch * sc, dtype=torch.float32, device=DEV)
    am = torch.zeros(batch * sc, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm_strided_batched(0, nat.SEMIRING[sr], 0, 0, _p(ta), _p(tb), _p(c), _p(am),
                                          batch, m, n, k, sa, sb, sc, None))
    torch.cuda.synchronize()
    c_np, am_np = c.cpu().numpy(), am.cpu().numpy()
    for t in range(batch):
        at = a[t * sa: t * sa + m * k].reshape(m, k)
        bt = b[t * sb: t * sb + k * n].reshape(k, n)
        c_ref, am_ref = oracle.gemm(sr, at, bt)
        assert_exact(c_np[t * sc: t * sc + m * n].reshape(m, n),
                     am_np[t * sc: t * sc + m * n].reshape(m, n), c_ref, am_ref)


def test_device_out_of_range_is_dimension_mismatch():
    from tropical_gemm import _native as nat

    lib = nat.load()
    n = nat.device_count()
    t = torch.zeros(16, device=DEV)
    rc = lib.tg_gemm(n + 3, 0, 0, 0, _p(t), _p(t), _p(t), None, 2, 2, 2, None)
    assert rc == nat.TG_ERR_DIMENSION_MISMATCH and "not available" in nat.last_error()


def test_context_and_memory_entry_points():
    from tropical_gemm import _native as nat

    lib = nat.load()
    nat.check(lib.tg_context_init(0))
    buf = ctypes.create_string_buffer(256)
    nat.check(lib.tg_device_name(0, buf, 256))
    assert b"gfx950" in buf.value
    ptr = ctypes.c_void_p()
    nat.check(lib.tg_malloc(0, ctypes.byref(ptr), 4096))
    host = np.arange(1024, dtype=np.float32)
    back = np.zeros_like(host)
    nat.check(lib.tg_memcpy_htod(0, ptr, host.ctypes.data_as(ctypes.c_void_p), host.nbytes))
    nat.check(lib.tg_memset_zero(0, ptr, 100, None))
    nat.check(lib.tg_synchronize(0))
    nat.check(lib.tg_memcpy_dtoh(0, back.ctypes.data_as(ctypes.c_void_p), ptr, host.nbytes))
    assert np.all(back[:25] == 0) and np.array_equal(back[25:], host[25:])
    nat.check(lib.tg_free(0, ptr))


# ---------------------------------------------------------------------------
# Full-tile shapes: 32-bit problems with M % 64 == 0, N % 128 == 0 and
# K % 32 == 0 take the direct-to-LDS kernel; these pin it to the oracle.
# ---------------------------------------------------------------------------

# K <= 192 resolves argmax in chunks of 8, K <= 768 in chunks of 16, else 32.
ALIGNED_SHAPES = [(64, 32, 128), (128, 160, 256), (192, 512, 256), (64, 768, 128),
                  (320, 1024, 384), (64, 4096, 128)]


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_full_tile_shapes(sr, dt):
    rng = np.random.default_rng(300 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in ALIGNED_SHAPES:
        print(f"[case] full-tile {sr} {dt} m={m} k={k} n={n}", flush=True)
        a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        c_ref, am_ref = oracle.gemm(sr, a, b)
        c, am = gpu_gemm(sr, a, b, True)
        assert_exact(c, am, c_ref, am_ref)
        c, _ = gpu_gemm(sr, a, b, False)
        assert_exact(c, None, c_ref, None)


# Value-only tile shapes chosen by how the tiles fill the resident slots of
# the 256 CUs: 64 x 128 tiles where 64 x 64 tiles would make exactly one
# round (1024 tiles), 128 x 128 tiles for exactly one round of their own
# (512 tiles).  The oracle checks a sample of rows (rows are independent).
VALUE_TILE_CASES = [
    ("maxplus", "f32", 2048, 2048, 256, "dl_4x8"),
    ("minplus", "f32", 2000, 2048, 160, "dl_4x8"),  # partial last row tile
    ("maxmul", "f32", 1024, 4096, 96, "dl_4x8"),
    ("maxplus", "i32", 2048, 2048, 128, "dl_4x8"),
    ("minplus", "i32", 2048, 2048, 256, "dl_4x8"),
    ("maxmul", "i32", 1024, 4096, 64, "dl_4x8"),
    ("minplus", "f32", 2048, 4096, 512, "dl_8x8_cl32"),
    ("maxplus", "f32", 2000, 4000, 256, "dl_8x8_cl32"),  # partial row and column tiles
]


@pytest.mark.parametrize("sr,dt,m,n,k,path", VALUE_TILE_CASES,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}x{c[3]}x{c[4]}-{c[5]}" for c in VALUE_TILE_CASES])
def test_value_only_tile_shapes(sr, dt, m, n, k, path):
    nat = _nat()
    assert nat.gemm_plan(sr, dt, m, n, k, False) == path
    print(f"[case] value-only tiles {sr} {dt} {m}x{n}x{k} {path}", flush=True)
    rng = np.random.default_rng(m + n + k)
    dtype = tc.NP_DTYPES[dt]
    a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
    b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
    c, _ = gpu_gemm(sr, a, b, False)
    rows = np.unique(np.concatenate([np.arange(0, m, 61), [63, 64, m - 1]]))
    c_ref, _ = oracle.gemm(sr, a[rows], b)
    assert_exact(c[rows], None, c_ref, None)


def test_value_only_wide_tiles_batched():
    """Four 1024 x 1024 items make one round of 64 x 64 tiles together, so
    the batch runs on 64 x 128 tiles (blockIdx.z per item)."""
    from tropical_gemm import ops

    nat = _nat()
    batch, m, n, k = 4, 1024, 1024, 256
    assert nat.gemm_plan("maxplus", "f32", m, n, k, False, batch=batch,
                         strides=(m * k, k * n, m * n)) == "dl_4x8"
    rng = np.random.default_rng(404)
    a = np.round(rng.standard_normal((batch, m, k)) * 4).astype(np.float32) / 4 + 0.0625
    b = np.round(rng.standard_normal((batch, k, n)) * 4).astype(np.float32) / 4 + 0.0625
    print("[case] value-only 64x128 tiles, batch 4", flush=True)
    c, _ = ops.gemm_batched("maxplus", torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV),
                            False)
    torch.cuda.synchronize()
    c = c.cpu().numpy()
    rows = np.array([0, 1, 63, 64, 500, m - 1])
    for z in range(batch):
        c_ref, _ = oracle.gemm("maxplus", a[z][rows], b[z])
        np.testing.assert_array_equal(tc.bits(c[z][rows]), tc.bits(c_ref))


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("k", [96, 320, 1056])
def test_full_tile_heavy_ties(sr, dt, k):
    rng = np.random.default_rng(78)
    dtype = tc.NP_DTYPES[dt]
    a = rng.integers(0, 3, size=(128, k)).astype(dtype)
    b = rng.integers(0, 3, size=(k, 256)).astype(dtype)
    c, am = gpu_gemm(sr, a, b)
    assert_exact(c, am, *oracle.gemm(sr, a, b))


def test_full_tile_special_values():
    rng = np.random.default_rng(5)
    a = rng.standard_normal((128, 256)).astype(np.float32)
    b = rng.standard_normal((256, 256)).astype(np.float32)
    a[rng.random(a.shape) < 0.3] = np.inf
    b[rng.random(b.shape) < 0.3] = np.inf
    assert_exact(*gpu_gemm("minplus", a, b), *oracle.gemm("minplus", a, b))
    a2 = np.where(np.isinf(a), -np.inf, a).astype(np.float32)
    b2 = np.where(np.isinf(b), -np.inf, b).astype(np.float32)
    a2[5, :] = -np.inf
    c, am = gpu_gemm("maxplus", a2, b2)
    assert_exact(c, am, *oracle.gemm("maxplus", a2, b2))
    assert np.all(np.isneginf(c[5])) and np.all(am[5] == 0)
    a3 = rng.integers(-2, 3, size=(64, 96)).astype(np.float32)
    b3 = rng.integers(-2, 3, size=(96, 128)).astype(np.float32)
    assert_exact(*gpu_gemm("maxmul", a3, b3), *oracle.gemm("maxmul", a3, b3))
    # signed zeros: -0 at k=0 ties +0 later; the first occurrence wins
    z = np.zeros((64, 64), np.float32)
    z[:, 0] = -0.0
    bz = np.full((64, 128), -1.0, np.float32)
    bz[0, :] = -0.0
    bz[40, :] = 0.0
    c, am = gpu_gemm("maxplus", z, bz)
    assert_exact(c, am, *oracle.gemm("maxplus", z, bz))
    assert np.all(np.signbit(c)) and np.all(am == 0)


def test_full_tile_strided_batched():
    from tropical_gemm import _native as nat

    lib = nat.load()
    rng = np.random.default_rng(13)
    batch, m, k, n = 3, 64, 96, 128
    sa, sb, sc = m * k + 4, k * n + 8, m * n + 12
    a = rng.standard_normal(batch * sa).astype(np.float32)
    b = rng.standard_normal(batch * sb).astype(np.float32)
    ta, tb = _dev(a), _dev(b)
    c = torch.zeros(batch * sc, dtype=torch.float32, device=DEV)
    am = torch.zeros(batch * sc, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm_strided_batched(0, nat.SEMIRING["maxplus"], 0, 0, _p(ta), _p(tb), _p(c),
                                          _p(am), batch, m, n, k, sa, sb, sc, None))
    torch.cuda.synchronize()
    c_np, am_np = c.cpu().numpy(), am.cpu().numpy()
    for t in range(batch):
        at = a[t * sa: t * sa + m * k].reshape(m, k)
        bt = b[t * sb: t * sb + k * n].reshape(k, n)
        assert_exact(c_np[t * sc: t * sc + m * n].reshape(m, n),
                     am_np[t * sc: t * sc + m * n].reshape(m, n), *oracle.gemm("maxplus", at, bt))


# Argmax problems with K > 768 and at least 1536 tiles of 64 x 128 take the
# wide-tile kernel.
WIDE_SHAPES = [(3072, 800, 4096), (1536, 1024, 8192)]


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_wide_tile_argmax(sr, dt):
    rng = np.random.default_rng(400 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in WIDE_SHAPES:
        print(f"[case] wide-tile {sr} {dt} m={m} k={k} n={n}", flush=True)
        if dt == "i32":
            a = rng.integers(-5, 6, size=(m, k)).astype(dtype)  # many ties
            b = rng.integers(-5, 6, size=(k, n)).astype(dtype)
        else:
            a = tc.rng_matrix(rng, dtype, (m, k))
            b = tc.rng_matrix(rng, dtype, (k, n))
        c, am = gpu_gemm(sr, a, b, True)
        assert_exact(c, am, *oracle.gemm(sr, a, b))


def test_wide_tile_argmax_batched():
    from tropical_gemm import ops

    rng = np.random.default_rng(41)
    a = rng.standard_normal((12, 512, 800)).astype(np.float32)
    b = rng.standard_normal((12, 800, 2048)).astype(np.float32)
    c, am = ops.gemm_batched("minplus", _dev(a), _dev(b), True)
    c, am = c.cpu().numpy(), am.cpu().numpy()
    for t in range(12):
        assert_exact(c[t], am[t], *oracle.gemm("minplus", a[t], b[t]))


# Argmax problems with K in {64, 96, 128} and full 64 x 64 tiles take the
# K-resident kernel (whole K panel in LDS, argmax resolved from LDS).
KRES_SHAPES = [(64, 64, 64), (128, 96, 192), (256, 128, 128), (192, 128, 320)]


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_k_resident_argmax(sr, dt):
    rng = np.random.default_rng(500 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in KRES_SHAPES:
        print(f"[case] k-resident {sr} {dt} m={m} k={k} n={n}", flush=True)
        a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        assert_exact(*gpu_gemm(sr, a, b, True), *oracle.gemm(sr, a, b))
        # Heavy ties: values in {0,1,2} put equal maxima in many chunks.
        a = rng.integers(0, 3, size=(m, k)).astype(dtype)
        b = rng.integers(0, 3, size=(k, n)).astype(dtype)
        for api in ("alloc", "ws"):
            assert_exact(*gpu_gemm(sr, a, b, True, api=api), *oracle.gemm(sr, a, b))


def test_k_resident_viterbi_shape_and_batches():
    from tropical_gemm import ops

    rng = np.random.default_rng(51)
    # Viterbi-like: emission scores in [-1000, 1000], transitions in [-50, 0].
    a = rng.integers(-1000, 1001, size=(4096, 128)).astype(np.int32)
    b = rng.integers(-50, 1, size=(128, 128)).astype(np.int32)
    c, am = gpu_gemm("maxplus", a, b, True)
    assert_exact(c, am, *oracle.gemm("maxplus", a, b))
    # Column-major storage maps onto the same kernel with the operands swapped.
    c, am = gpu_gemm("maxplus", a[:128], b, True, layout="col")
    assert_exact(c, am, *oracle.gemm("maxplus", a[:128], b))
    a3 = rng.standard_normal((5, 128, 64)).astype(np.float32)
    b3 = rng.standard_normal((5, 64, 192)).astype(np.float32)
    c3, am3 = ops.gemm_batched("minplus", _dev(a3), _dev(b3), True)
    c3, am3 = c3.cpu().numpy(), am3.cpu().numpy()
    for t in range(5):
        assert_exact(c3[t], am3[t], *oracle.gemm("minplus", a3[t], b3[t]))


def test_k_resident_special_values():
    rng = np.random.default_rng(52)
    a = rng.standard_normal((128, 128)).astype(np.float32)
    b = rng.standard_normal((128, 64)).astype(np.float32)
    a[rng.random(a.shape) < 0.3] = np.inf
    b[rng.random(b.shape) < 0.3] = np.inf
    a[7, :] = np.inf  # row never beats the MinPlus zero: +inf, argmax 0
    c, am = gpu_gemm("minplus", a, b)
    assert_exact(c, am, *oracle.gemm("minplus", a, b))
    assert np.all(np.isposinf(c[7])) and np.all(am[7] == 0)
    # MaxMul: products <= 0 never beat the zero.
    a3 = rng.integers(-2, 3, size=(64, 64)).astype(np.float32)
    b3 = rng.integers(-2, 3, size=(64, 64)).astype(np.float32)
    assert_exact(*gpu_gemm("maxmul", a3, b3), *oracle.gemm("maxmul", a3, b3))
    # Signed zeros: -0 at k=0 ties +0 later in the same and in later chunks.
    z = np.zeros((64, 96), np.float32)
    z[:, 0] = -0.0
    bz = np.full((96, 64), -1.0, np.float32)
    bz[0, :] = -0.0
    bz[3, :] = 0.0
    bz[70, :] = 0.0
    c, am = gpu_gemm("maxplus", z, bz)
    assert_exact(c, am, *oracle.gemm("maxplus", z, bz))
    assert np.all(np.signbit(c)) and np.all(am == 0)


# The B^T workspace: exactly tg_gemm_workspace_size bytes must suffice for
# both layouts (column-major calls swap the operands, so the kernel's B is A
# and needs k x m elements).  A guard region after the workspace must be left
# untouched.
@pytest.mark.parametrize("layout", ["row", "col"])
@pytest.mark.parametrize("shape", [(45, 77, 29), (29, 77, 45), (130, 64, 64), (64, 64, 130),
                                   (256, 96, 128)])
def test_workspace_bound_and_guard(layout, shape):
    nat = _nat()
    lib = nat.load()
    m, k, n = shape
    rng = np.random.default_rng(61)
    a = rng.integers(-20, 21, size=(m, k)).astype(np.float32)
    b = rng.integers(-20, 21, size=(k, n)).astype(np.float32)
    c_ref, am_ref = oracle.gemm("maxplus", a, b)
    if layout == "col":
        ta, tb = _dev(np.asfortranarray(a).T.copy()), _dev(np.asfortranarray(b).T.copy())
    else:
        ta, tb = _dev(a), _dev(b)
    ws_bytes = lib.tg_gemm_workspace_size(0, 1, m, n, k, 1)
    assert ws_bytes >= k * max(m, n) * 4
    guard = 65536
    ws = torch.full((ws_bytes + guard,), 0xA5, dtype=torch.uint8, device=DEV)
    c = torch.empty(m * n, dtype=torch.float32, device=DEV)
    am = torch.empty(m * n, dtype=torch.int32, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.check(lib.tg_gemm_ws(0, 0, 0, nat.LAYOUT[layout], _p(ta), _p(tb), _p(c), _p(am), m, n, k,
                             _p(ws), ws_bytes, stream))
    torch.cuda.synchronize()
    assert bool(torch.all(ws[ws_bytes:] == 0xA5)), "workspace overrun"
    if layout == "col":
        c_np, am_np = c.cpu().numpy().reshape(n, m).T, am.cpu().numpy().reshape(n, m).T
    else:
        c_np, am_np = c.cpu().numpy().reshape(m, n), am.cpu().numpy().reshape(m, n)
    assert_exact(c_np, am_np, c_ref, am_ref)
    # Strided batches of the same product: the workspace holds one B^T each.
    batch = 3
    ta3 = ta.reshape(-1).repeat(batch)
    tb3 = tb.reshape(-1).repeat(batch)
    ws_bytes = lib.tg_gemm_workspace_size(0, batch, m, n, k, 1)
    ws = torch.full((ws_bytes + guard,), 0xA5, dtype=torch.uint8, device=DEV)
    c3 = torch.empty(batch * m * n, dtype=torch.float32, device=DEV)
    am3 = torch.empty(batch * m * n, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm_strided_batched_ws(0, 0, 0, nat.LAYOUT[layout], _p(ta3), _p(tb3), _p(c3),
                                             _p(am3), batch, m, n, k, m * k, k * n, m * n, _p(ws),
                                             ws_bytes, stream))
    torch.cuda.synchronize()
    assert bool(torch.all(ws[ws_bytes:] == 0xA5)), "batched workspace overrun"
    for t in range(batch):
        ct = c3[t * m * n:(t + 1) * m * n].cpu().numpy()
        at = am3[t * m * n:(t + 1) * m * n].cpu().numpy()
        if layout == "col":
            ct, at = ct.reshape(n, m).T, at.reshape(n, m).T
        else:
            ct, at = ct.reshape(m, n), at.reshape(m, n)
        assert_exact(ct, at, c_ref, am_ref)


# The K-resident kernel's three i32 paths, chosen per workgroup from the
# magnitudes in its panels: f32 keys (all |x| < 2^15), i32 keys (< 2^22) and
# the chunked path (anything larger, including wraparound).  The calls pass
# the documented minimum workspace (k x max(m, n)), which the K-resident
# kernel does not need at all.
@pytest.mark.parametrize("sr", ["maxplus", "minplus", "maxmul"])
def test_k_resident_integer_paths(sr):
    rng = np.random.default_rng(53)
    m, k, n = 256, 128, 128
    api = "min"
    cases = {
        "f32-key boundary": (rng.choice([-32768, -32767, 0, 32766, 32767], size=(m, k)),
                             rng.choice([-32768, 32767, 1, -1], size=(k, n))),
        "i32-key": (rng.integers(-(1 << 21), 1 << 21, size=(m, k)),
                    rng.integers(-(1 << 21), 1 << 21, size=(k, n))),
        "i32-key ties": (rng.integers(0, 3, size=(m, k)) * 40000,
                         rng.integers(0, 3, size=(k, n)) * 40000),
        "chunked wraparound": (rng.integers(2**31 - 60, 2**31 - 1, size=(m, k)),
                               rng.integers(-5, 60, size=(k, n))),
    }
    for name, (a, b) in cases.items():
        print(f"[case] k-resident {sr} i32 {name}", flush=True)
        a = a.astype(np.int32)
        b = b.astype(np.int32)
        assert_exact(*gpu_gemm(sr, a, b, True, api=api), *oracle.gemm(sr, a, b))
    # One workgroup's panel (rows 64..127) holds a large value: that workgroup
    # takes the chunked path, the others keep the key paths.
    a = rng.integers(-1000, 1001, size=(m, k)).astype(np.int32)
    b = rng.integers(-50, 1, size=(k, n)).astype(np.int32)
    a[100, 7] = 1 << 24
    assert_exact(*gpu_gemm(sr, a, b, True, api=api), *oracle.gemm(sr, a, b))
    a[100, 7] = 1 << 17
    assert_exact(*gpu_gemm(sr, a, b, True, api=api), *oracle.gemm(sr, a, b))


def _strided_batched(sr, items, gap_a=24, gap_c=40):
    """Run tg_gemm_strided_batched_ws on a list of (A, B) with gaps after
    every A and C; return the per-item (C, argmax) and check the gaps."""
    nat = _nat()
    lib = nat.load()
    m, k = items[0][0].shape
    n = items[0][1].shape[1]
    batch = len(items)
    dt = DT_NAME[items[0][0].dtype]
    sa, sb, sc = m * k + gap_a, k * n, m * n + gap_c
    ha = np.zeros(batch * sa, items[0][0].dtype)
    hb = np.zeros(batch * sb, items[0][0].dtype)
    for t, (x, y) in enumerate(items):
        ha[t * sa:t * sa + m * k] = x.ravel()
        hb[t * sb:t * sb + k * n] = y.ravel()
    ta, tb = _dev(ha), _dev(hb)
    c3 = torch.full((batch * sc,), 7, dtype=TORCH_DT[items[0][0].dtype], device=DEV)
    am3 = torch.full((batch * sc,), 7, dtype=torch.int32, device=DEV)
    ws_bytes = lib.tg_gemm_workspace_size(nat.DTYPE[dt], batch, m, n, k, 1)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.check(lib.tg_gemm_strided_batched_ws(0, nat.SEMIRING[sr], nat.DTYPE[dt], nat.LAYOUT["row"],
                                             _p(ta), _p(tb), _p(c3), _p(am3), batch, m, n, k, sa,
                                             sb, sc, _p(ws), ws_bytes, stream))
    torch.cuda.synchronize()
    cv, iv = c3.cpu().numpy(), am3.cpu().numpy()
    out = []
    for t in range(batch):
        assert np.all(cv[t * sc + m * n:(t + 1) * sc] == 7), "gap after C overwritten"
        assert np.all(iv[t * sc + m * n:(t + 1) * sc] == 7), "gap after argmax overwritten"
        out.append((cv[t * sc:t * sc + m * n].reshape(m, n), iv[t * sc:t * sc + m * n].reshape(m, n)))
    return out


# The 64 x 128 K-resident kernel (i32 MaxPlus/MinPlus, N a multiple of
# 128): batch items change the resident B panel; a row tile that leaves the
# f32-key range turns the B panel raw for the chunked path and the next tile
# turns it back into keys; a batch item whose B panel is out of range runs
# every tile chunked.
@pytest.mark.parametrize("sr", ["maxplus", "minplus"])
def test_k_resident_wide_tiles(sr):
    rng = np.random.default_rng(57 + (sr == "minplus"))
    for (m, k, n, batch) in [(256, 64, 256, 1), (512, 96, 128, 3), (384, 128, 384, 2),
                             (4096, 128, 128, 2), (4160, 128, 128, 2)]:
        print(f"[case] k-resident 64x128 {sr} m={m} k={k} n={n} batch={batch}", flush=True)
        items = []
        for t in range(batch):
            a = rng.integers(-1000, 1001, size=(m, k))
            b = rng.integers(-50, 1, size=(k, n))
            a[70 + t, 3] = 40000  # row tile 1 leaves the key range
            if t == 1:
                b[3, 5] = 1 << 20  # this item's whole B panel does
            items.append((a.astype(np.int32), b.astype(np.int32)))
        for (c, am), (a, b) in zip(_strided_batched(sr, items), items):
            assert_exact(c, am, *oracle.gemm(sr, a, b))
        for name, lo, hi in (("ties", 0, 3), ("wraparound", 2**31 - 60, 2**31 - 1)):
            a = rng.integers(lo, hi, size=(m, k)).astype(np.int32)
            b = rng.integers(0 if name == "ties" else -5, 3 if name == "ties" else 60,
                             size=(k, n)).astype(np.int32)
            for api in ("alloc", "min"):
                assert_exact(*gpu_gemm(sr, a, b, True, api=api), *oracle.gemm(sr, a, b))


@pytest.mark.parametrize("sr", ["maxplus", "minplus"])
def test_k_resident_several_tiles_per_workgroup(sr):
    """2048 row tiles over the persistent grid (several per workgroup):
    tiles that fail the key-range vote next to tiles that pass it, in both
    orders within one workgroup, plus a batch of two with the second item's B
    panel out of range."""
    rng = np.random.default_rng(59 + (sr == "minplus"))
    m, k, n = 131072, 128, 128
    a = rng.integers(-1000, 1001, size=(m, k))
    b = rng.integers(-50, 1, size=(k, n))
    for row in (70, 128 * 513 + 5, 128 * 900 + 127, 128 * 901):
        a[row, row % k] = -40000
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    print(f"[case] k-resident {sr} m={m} scattered out-of-range rows", flush=True)
    assert_exact(*gpu_gemm(sr, a, b, True, api="min"), *oracle.gemm(sr, a, b))
    b2 = b.copy()
    b2[100, 0] = 1 << 17
    items = [(a[:65536], b), (a[65536:], b2)]
    print(f"[case] k-resident {sr} batch of two, second B out of range", flush=True)
    for (c, am), (x, y) in zip(_strided_batched(sr, items), items):
        assert_exact(c, am, *oracle.gemm(sr, x, y))


# The wave-private K-resident kernel (tg_gemm_kresw: M a multiple of 16, N a
# multiple of 128 up to 16 column tiles): row counts that are not multiples
# of 64, several column tiles, fewer row tiles than waves, a wave tile that
# leaves the key range in its last k-tile (the exact fallback after three
# k-tiles on keys), a batch item whose B panel leaves it, and the tile after
# a fallback back on keys.
@pytest.mark.parametrize("sr", ["maxplus", "minplus"])
def test_k_resident_wave_tiles(sr):
    nat = _nat()
    rng = np.random.default_rng(61 + (sr == "minplus"))
    for (m, k, n, batch) in [(16, 64, 128, 1), (48, 96, 256, 2), (4112, 128, 384, 3),
                             (2064, 128, 2048, 1)]:
        assert nat.gemm_plan(sr, "i32", m, n, k, True) == "kresw"
        print(f"[case] k-resident wave tiles {sr} m={m} k={k} n={n} batch={batch}", flush=True)
        items = []
        for t in range(batch):
            a = rng.integers(-1000, 1001, size=(m, k))
            b = rng.integers(-50, 1, size=(k, n))
            a[min(m - 1, 17 + t), k - 1] = 40000  # a wave tile's last k-tile leaves the key range
            if t == 1:
                b[k - 1, n - 1] = -(1 << 20)  # this item's whole B panel does
            items.append((a.astype(np.int32), b.astype(np.int32)))
        if batch == 1:
            a, b = items[0]
            for api in ("alloc", "min"):
                assert_exact(*gpu_gemm(sr, a, b, True, api=api), *oracle.gemm(sr, a, b))
        else:
            for (c, am), (a, b) in zip(_strided_batched(sr, items), items):
                assert_exact(c, am, *oracle.gemm(sr, a, b))
    # Wider than 16 column tiles: the 64 x 128 kernel (tg_gemm_kres8) keeps
    # these, with its key path and its chunked fallback.
    m, k, n = 192, 96, 128 * 17
    assert nat.gemm_plan(sr, "i32", m, n, k, True) == "kres8"
    a = rng.integers(-1000, 1001, size=(m, k))
    b = rng.integers(-50, 1, size=(k, n))
    a[70, 5] = 40000
    a, b = a.astype(np.int32), b.astype(np.int32)
    print(f"[case] k-resident 64x128 {sr} m={m} k={k} n={n}", flush=True)
    assert_exact(*gpu_gemm(sr, a, b, True), *oracle.gemm(sr, a, b))
    # Ties at the f32-key boundary and wraparound through the exact path.
    m, k, n = 272, 128, 256
    for name, a, b in (
        ("key boundary ties", rng.choice([-32767, 0, 32767], size=(m, k)),
         rng.choice([-32767, 0, 32767], size=(k, n))),
        ("wraparound", rng.integers(2**31 - 60, 2**31 - 1, size=(m, k)),
         rng.integers(-5, 60, size=(k, n))),
    ):
        print(f"[case] k-resident wave tiles {sr} {name}", flush=True)
        a = a.astype(np.int32)
        b = b.astype(np.int32)
        assert_exact(*gpu_gemm(sr, a, b, True), *oracle.gemm(sr, a, b))


# Short-K i32 argmax over ragged and full-tile shapes (K in {32, 64, 96,
# 128}, N a multiple of 64, M anything): the key-range boundary, ties,
# wraparound, one row or one B entry just outside the f32-key range, and rows
# that never beat the tropical zero.
SHORT_K_SHAPES = [(1, 32, 64), (63, 64, 128), (200, 96, 192), (4113, 128, 128), (130, 128, 256),
                  (77, 64, 320), (256, 128, 128)]


@pytest.mark.parametrize("sr", ["maxplus", "minplus"])
def test_short_k_integer_argmax(sr):
    rng = np.random.default_rng(54 + (sr == "minplus"))
    for (m, k, n) in SHORT_K_SHAPES:
        cases = {
            "viterbi": (rng.integers(-1000, 1001, size=(m, k)), rng.integers(-50, 1, size=(k, n))),
            "key boundary": (rng.choice([-32768, -32767, 0, 32766, 32767], size=(m, k)),
                             rng.choice([-32768, 32767, 1, -1], size=(k, n))),
            "ties": (rng.integers(0, 3, size=(m, k)), rng.integers(0, 3, size=(k, n))),
            "wraparound": (rng.integers(2**31 - 60, 2**31 - 1, size=(m, k)),
                           rng.integers(-5, 60, size=(k, n))),
        }
        # One row just outside the f32-key range.
        a = rng.integers(-1000, 1001, size=(m, k))
        a[m // 2, k - 1] = 32768
        cases["one wave chunked"] = (a, rng.integers(-50, 1, size=(k, n)))
        # One B entry just outside it.
        b = rng.integers(-50, 1, size=(k, n))
        b[k // 3, n - 1] = -32769
        cases["one block chunked"] = (rng.integers(-1000, 1001, size=(m, k)), b)
        # Rows that never beat the tropical zero keep it, with argmax 0.
        a = rng.integers(-1000, 1001, size=(m, k))
        zero = -(2**31) if sr == "maxplus" else 2**31 - 1
        a[0, :] = zero
        cases["zero row"] = (a, np.zeros((k, n), np.int64))
        for name, (a, b) in cases.items():
            print(f"[case] short-k {sr} m={m} k={k} n={n} {name}", flush=True)
            a = a.astype(np.int32)
            b = b.astype(np.int32)
            ref = oracle.gemm(sr, a, b)
            for api in ("alloc", "ws", "min"):
                assert_exact(*gpu_gemm(sr, a, b, True, api=api), *ref)


def test_short_k_integer_layouts_batches_and_guard():
    """Column-major calls (the kernels' N is m), strided batches with gaps in
    which one item leaves the f32-key range, and a guard after exactly
    tg_gemm_workspace_size bytes of workspace."""
    nat = _nat()
    lib = nat.load()
    rng = np.random.default_rng(56)
    a = rng.integers(-1000, 1001, size=(128, 64)).astype(np.int32)
    b = rng.integers(-1000, 1001, size=(64, 1000)).astype(np.int32)
    c, am = gpu_gemm("maxplus", a, b, True, layout="col")
    assert_exact(c, am, *oracle.gemm("maxplus", a, b))

    batch, m, k, n = 3, 300, 96, 192
    gap_a, gap_c = 40, 24
    items = [(rng.integers(-1000, 1001, size=(m, k)), rng.integers(-50, 1, size=(k, n)))
             for _ in range(batch)]
    items[1][0][5, 5] = 1 << 20  # this item's first row tile leaves the f32-key range
    sa, sb, sc = m * k + gap_a, k * n, m * n + gap_c
    ha = np.zeros(batch * sa, np.int32)
    hb = np.zeros(batch * sb, np.int32)
    for t, (x, y) in enumerate(items):
        ha[t * sa:t * sa + m * k] = x.ravel()
        hb[t * sb:t * sb + k * n] = y.ravel()
    for sr in ("maxplus", "minplus"):
        ws_bytes = lib.tg_gemm_workspace_size(nat.DTYPE["i32"], batch, m, n, k, 1)
        guard = 65536
        ws = torch.full((ws_bytes + guard,), 0xA5, dtype=torch.uint8, device=DEV)
        c3 = torch.full((batch * sc,), 7, dtype=torch.int32, device=DEV)
        am3 = torch.full((batch * sc,), 7, dtype=torch.int32, device=DEV)
        ta, tb = _dev(ha), _dev(hb)
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        nat.check(lib.tg_gemm_strided_batched_ws(0, nat.SEMIRING[sr], nat.DTYPE["i32"],
                                                 nat.LAYOUT["row"], _p(ta), _p(tb), _p(c3),
                                                 _p(am3), batch, m, n, k, sa, sb, sc, _p(ws),
                                                 ws_bytes, stream))
        torch.cuda.synchronize()
        assert bool(torch.all(ws[ws_bytes:] == 0xA5)), "workspace overrun"
        cv, iv = c3.cpu().numpy(), am3.cpu().numpy()
        for t, (x, y) in enumerate(items):
            assert_exact(cv[t * sc:t * sc + m * n].reshape(m, n),
                         iv[t * sc:t * sc + m * n].reshape(m, n),
                         *oracle.gemm(sr, x.astype(np.int32), y.astype(np.int32)))
            assert np.all(cv[t * sc + m * n:(t + 1) * sc] == 7), "gap after C overwritten"
            assert np.all(iv[t * sc + m * n:(t + 1) * sc] == 7), "gap after argmax overwritten"


# Split K: full-tile 32-bit problems with few 64 x 64 tiles run K in slices
# (up to 1024 workgroups, slices of >= 256 k) and merge the per-slice
# (value, first k) partials; ties go to the earlier slice.
SPLIT_SHAPES = [(64, 4096, 64), (128, 512, 128), (256, 8192, 256), (192, 1536, 320)]


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_split_k(sr, dt):
    nat = _nat()
    lib = nat.load()
    rng = np.random.default_rng(600 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n) in SPLIT_SHAPES:
        full = lib.tg_gemm_workspace_size(nat.DTYPE[dt], 1, m, n, k, 1)
        assert full > k * max(m, n) * 4, "split-K partials must be part of the workspace size"
        print(f"[case] split-k {sr} {dt} m={m} k={k} n={n}", flush=True)
        a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        c_ref, am_ref = oracle.gemm(sr, a, b)
        for api in ("alloc", "ws"):
            assert_exact(*gpu_gemm(sr, a, b, True, api=api), c_ref, am_ref)
            c, _ = gpu_gemm(sr, a, b, False, api=api)
            assert_exact(c, None, c_ref, None)
        # Equal maxima in many slices: the first k must win.
        a = rng.integers(0, 3, size=(m, k)).astype(dtype)
        b = rng.integers(0, 3, size=(k, n)).astype(dtype)
        assert_exact(*gpu_gemm(sr, a, b, True), *oracle.gemm(sr, a, b))


def test_split_k_signed_zero_and_infinities():
    # -0 at k = 0 (slice 0) ties +0 at k = 3000 (a later slice): -0 / index 0.
    m, k, n = 64, 4096, 64
    a = np.zeros((m, k), np.float32)
    a[:, 0] = -0.0
    b = np.full((k, n), -1.0, np.float32)
    b[0, :] = -0.0
    b[3000, :] = 0.0
    c, am = gpu_gemm("maxplus", a, b)
    assert_exact(c, am, *oracle.gemm("maxplus", a, b))
    assert np.all(np.signbit(c)) and np.all(am == 0)
    # +inf entries (MinPlus "no edge") with rows that are +inf in every slice.
    rng = np.random.default_rng(62)
    a = (rng.random((m, k)) * 100).astype(np.float32)
    b = (rng.random((k, n)) * 100).astype(np.float32)
    a[rng.random(a.shape) < 0.3] = np.inf
    b[rng.random(b.shape) < 0.3] = np.inf
    a[5, :] = np.inf
    c, am = gpu_gemm("minplus", a, b)
    assert_exact(c, am, *oracle.gemm("minplus", a, b))
    assert np.all(np.isposinf(c[5])) and np.all(am[5] == 0)


def test_split_k_minimum_workspace_and_batches():
    nat = _nat()
    lib = nat.load()
    rng = np.random.default_rng(63)
    m, k, n = 128, 2048, 128
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c_ref, am_ref = oracle.gemm("maxplus", a, b)
    # A workspace of just the B^T staging runs the product unsplit.
    ws_min = k * n * 4
    ws = torch.empty(ws_min, dtype=torch.uint8, device=DEV)
    ta, tb = _dev(a), _dev(b)
    c = torch.empty(m * n, dtype=torch.float32, device=DEV)
    am = torch.empty(m * n, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm_ws(0, 0, 0, 0, _p(ta), _p(tb), _p(c), _p(am), m, n, k, _p(ws), ws_min,
                             None))
    torch.cuda.synchronize()
    assert_exact(c.cpu().numpy().reshape(m, n), am.cpu().numpy().reshape(m, n), c_ref, am_ref)
    # Strided batches with gaps between the outputs, split as one problem.
    from tropical_gemm import ops

    a3 = rng.standard_normal((3, 128, 1024)).astype(np.float32)
    b3 = rng.standard_normal((3, 1024, 64)).astype(np.float32)
    c3, am3 = ops.gemm_batched("maxplus", _dev(a3), _dev(b3), True)
    c3, am3 = c3.cpu().numpy(), am3.cpu().numpy()
    for t in range(3):
        assert_exact(c3[t], am3[t], *oracle.gemm("maxplus", a3[t], b3[t]))
    batch, sc = 3, 128 * 64 + 64
    ta3, tb3 = _dev(a3), _dev(b3)
    cc = torch.zeros(batch * sc, dtype=torch.float32, device=DEV)
    aa = torch.zeros(batch * sc, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm_strided_batched(0, 0, 0, 0, _p(ta3), _p(tb3), _p(cc), _p(aa), batch, 128,
                                          64, 1024, 128 * 1024, 1024 * 64, sc, None))
    torch.cuda.synchronize()
    cc, aa = cc.cpu().numpy(), aa.cpu().numpy()
    for t in range(batch):
        assert_exact(cc[t * sc: t * sc + 128 * 64].reshape(128, 64),
                     aa[t * sc: t * sc + 128 * 64].reshape(128, 64), *oracle.gemm("maxplus", a3[t], b3[t]))


# ---------------------------------------------------------------------------
# Short K (at most 32): the tiles kernel's exact mode, which tracks the index
# of every product (no chunk records, no resolve, no B^T staging) and writes
# four consecutive outputs per 16-byte store where the rows allow it.
# ---------------------------------------------------------------------------

EXACT_KS = [1, 2, 5, 8, 16, 31, 32, 33]


@pytest.mark.parametrize("dt", ["f32", "f64", "i32", "i64"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_exact_mode_short_k(sr, dt):
    """K up to 32 on both sides of the boundary (33 takes the chunked
    kernels), N a multiple of 4 (vector stores) or odd (element stores),
    random values and values in {0, 1, 2} (many maximisers per output)."""
    rng = np.random.default_rng(300 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for k in EXACT_KS:
        for (m, n) in [(200, 132), (77, 45), (129, 256)]:
            for ties in (False, True):
                print(f"[case] exact {sr} {dt} m={m} k={k} n={n} ties={ties}", flush=True)
                if ties:
                    a = rng.integers(0, 3, size=(m, k)).astype(dtype)
                    b = rng.integers(0, 3, size=(k, n)).astype(dtype)
                else:
                    a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
                    b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
                ref = oracle.gemm(sr, a, b)
                assert_exact(*gpu_gemm(sr, a, b, True, api="min"), *ref)
                c, _ = gpu_gemm(sr, a, b, False)
                assert_exact(c, None, ref[0], None)


def test_exact_mode_special_values_and_zero_rows():
    rng = np.random.default_rng(310)
    m, k, n = 96, 24, 136
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    a[rng.random(a.shape) < 0.2] = -np.inf
    b[rng.random(b.shape) < 0.2] = -np.inf
    a[3, :] = -np.inf  # never beats the zero: -inf with argmax 0
    c, am = gpu_gemm("maxplus", a, b)
    assert_exact(c, am, *oracle.gemm("maxplus", a, b))
    assert np.all(np.isneginf(c[3])) and np.all(am[3] == 0)
    ai = np.where(np.isinf(a), np.inf, a).astype(np.float32)
    bi = np.where(np.isinf(b), np.inf, b).astype(np.float32)
    assert_exact(*gpu_gemm("minplus", ai, bi), *oracle.gemm("minplus", ai, bi))
    # -0 at k = 0 ties +0 later: the first one (-0, index 0) stays.
    z = np.zeros((4, 9), np.float32)
    z[:, 0] = -0.0
    w = np.full((9, 8), -1.0, np.float32)
    w[0, :] = -0.0
    w[6, :] = 0.0
    c, am = gpu_gemm("maxplus", z, w)
    assert np.all(np.signbit(c)) and np.all(am == 0)
    # Integer wraparound.
    ia = rng.integers(2**31 - 60, 2**31 - 1, size=(70, 12)).astype(np.int32)
    ib = rng.integers(-5, 60, size=(12, 44)).astype(np.int32)
    for sr in tc.SEMIRINGS:
        assert_exact(*gpu_gemm(sr, ia, ib), *oracle.gemm(sr, ia, ib))


@pytest.mark.parametrize("dt", ["f32", "f64"])
def test_exact_mode_strided_batches_and_misaligned_outputs(dt):
    """Strided batches whose output stride keeps (sc = m*n + 4) or breaks
    (m*n + 1) 16-byte alignment of each item's rows, and a C / argmax pair
    that starts one element past an aligned address (element stores)."""
    nat = _nat()
    lib = nat.load()
    rng = np.random.default_rng(320)
    dtype = tc.NP_DTYPES[dt]
    d = nat.DTYPE[dt]
    batch, m, k, n = 3, 70, 20, 68
    for gap_c in (4, 1):
        print(f"[case] exact strided {dt} gap_c={gap_c}", flush=True)
        sa, sb, sc = m * k + 3, k * n + 5, m * n + gap_c
        a = tc.rng_matrix(rng, dtype, (batch * sa,), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (batch * sb,), -1000, 1000)
        ta, tb = _dev(a), _dev(b)
        c = torch.zeros(batch * sc, dtype=TORCH_DT[np.dtype(dtype)], device=DEV)
        am = torch.zeros(batch * sc, dtype=torch.int32, device=DEV)
        nat.check(lib.tg_gemm_strided_batched(0, nat.SEMIRING["maxplus"], d, 0, _p(ta), _p(tb),
                                              _p(c), _p(am), batch, m, n, k, sa, sb, sc, None))
        torch.cuda.synchronize()
        c_np, am_np = c.cpu().numpy(), am.cpu().numpy()
        for t in range(batch):
            ref = oracle.gemm("maxplus", a[t * sa:t * sa + m * k].reshape(m, k),
                              b[t * sb:t * sb + k * n].reshape(k, n))
            assert_exact(c_np[t * sc:t * sc + m * n].reshape(m, n),
                         am_np[t * sc:t * sc + m * n].reshape(m, n), *ref)
    print(f"[case] exact misaligned output {dt}", flush=True)
    a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
    b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
    ta, tb = _dev(a), _dev(b)
    c = torch.zeros(m * n + 1, dtype=TORCH_DT[np.dtype(dtype)], device=DEV)
    am = torch.zeros(m * n + 1, dtype=torch.int32, device=DEV)
    nat.check(lib.tg_gemm(0, nat.SEMIRING["minplus"], d, 0, _p(ta), _p(tb),
                          ctypes.c_void_p(c.data_ptr() + c.element_size()),
                          ctypes.c_void_p(am.data_ptr() + 4), m, n, k, None))
    torch.cuda.synchronize()
    assert_exact(c.cpu().numpy()[1:].reshape(m, n), am.cpu().numpy()[1:].reshape(m, n),
                 *oracle.gemm("minplus", a, b))


# ---------------------------------------------------------------------------
# Partial edge tiles in the direct-to-LDS kernels: M anything, N a multiple of
# 4 (whole 16-byte groups), K a multiple of 32.  The loads of a partial tile
# clamp into the matrix and the stores skip what lies outside it.
# ---------------------------------------------------------------------------

# The last three split K (few tiles, long K) with the full workspace and run
# unsplit with the minimum one.
PARTIAL_SHAPES = [(100, 64, 132, True), (65, 512, 68, True), (4100, 1024, 4100, True),
                  (4100, 1024, 4096, True), (1, 416, 4, True), (130, 96, 260, False),
                  (1, 32, 4, False), (4097, 640, 1028, False), (1000, 1024, 1000, True),
                  (70, 2048, 68, True), (70, 2048, 68, False)]


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_direct_to_lds_partial_tiles(sr, dt):
    rng = np.random.default_rng(400 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n, argmax) in PARTIAL_SHAPES:
        print(f"[case] partial tiles {sr} {dt} m={m} k={k} n={n} argmax={argmax}", flush=True)
        if sr == "maxmul" and dt == "f32":
            a = (1.0 - rng.random((m, k))).astype(dtype)
            b = (1.0 - rng.random((k, n))).astype(dtype)
        else:
            a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
            b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        ref = oracle.gemm(sr, a, b, with_argmax=argmax)
        for api in ("alloc", "ws", "min"):
            c, am = gpu_gemm(sr, a, b, argmax, api=api)
            assert_exact(c, am, ref[0], ref[1] if argmax else None)


def test_direct_to_lds_partial_tiles_batched_and_col_major():
    """Strided batches with gaps and partial tiles; a column-major call whose
    swapped operands make the kernel's M ragged."""
    rng = np.random.default_rng(410)
    items = [(rng.standard_normal((70, 256)).astype(np.float32),
              rng.standard_normal((256, 132)).astype(np.float32)) for _ in range(3)]
    print("[case] partial tiles batched", flush=True)
    for (c, am), (a, b) in zip(_strided_batched("maxplus", items), items):
        assert_exact(c, am, *oracle.gemm("maxplus", a, b))
    a = rng.standard_normal((132, 512)).astype(np.float32)
    b = rng.standard_normal((512, 70)).astype(np.float32)
    print("[case] partial tiles column-major", flush=True)
    c, am = gpu_gemm("minplus", a, b, True, layout="col")
    assert_exact(c, am, *oracle.gemm("minplus", a, b))
    # Column-major split K: the kernel's N is m (68), its M is n (70); the
    # workspace size covers both orientations.
    a = rng.standard_normal((68, 2048)).astype(np.float32)
    b = rng.standard_normal((2048, 70)).astype(np.float32)
    ref = oracle.gemm("maxplus", a, b)
    for api in ("alloc", "ws", "min"):
        print(f"[case] partial tiles column-major split K api={api}", flush=True)
        assert_exact(*gpu_gemm("maxplus", a, b, True, layout="col", api=api), *ref)


# K not a multiple of 32 (but of 4) in the direct-to-LDS kernels: the last
# k-tile is partial and the last argmax chunk may end past K.  Argmax cases
# have K above the exact mode's limit; "late" puts the maximum (and a tie) in
# the last, partial chunk.
RAGGED_K_SHAPES = [(130, 1000, 68, True), (65, 420, 132, True), (130, 100, 68, False),
                   (1, 36, 4, False), (4100, 1000, 4100, True), (257, 644, 260, False)]


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_direct_to_lds_ragged_k(sr, dt):
    rng = np.random.default_rng(420 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, k, n, argmax) in RAGGED_K_SHAPES:
        for late in (False, True):
            print(f"[case] ragged K {sr} {dt} m={m} k={k} n={n} argmax={argmax} late={late}",
                  flush=True)
            if sr == "maxmul" and dt == "f32":
                a = (1.0 - rng.random((m, k))).astype(dtype)
                b = (1.0 - rng.random((k, n))).astype(dtype)
            else:
                a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
                b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
            if late:
                big = {"maxplus": 5000, "minplus": -5000, "maxmul": 5000}[sr]
                a[:, k - 1] = big
                a[:, k - 3] = big
                b[k - 3] = np.abs(b[k - 3]) + 1  # at least 1: these products dominate
                b[k - 1] = b[k - 3]  # the same product at k-3 and k-1: the first wins
            ref = oracle.gemm(sr, a, b, with_argmax=argmax)
            c, am = gpu_gemm(sr, a, b, argmax, api="ws")
            assert_exact(c, am, ref[0], ref[1] if argmax else None)
            if argmax and late and not (sr == "maxmul" and dt == "i32"):
                assert np.all(am == k - 3)  # (i32 MaxMul: negative B can outweigh it)


# The short-K kernel (N % 4 == 0, K up to 32 with argmax and up to 63
# value-only): 32 x 256 tiles with 8 rows per wave for 32-bit types, 16 x 256
# with 4 rows for 64-bit ones, A read through scalar loads in 32-byte blocks.  Rows past M inside a wave, column quads past N,
# K around the 8-k blocks, wrapping i32 products, and strided batches whose
# A rows start at odd element offsets.
SHORTK_KERNEL_SHAPES = [(1, 4, 1), (5, 260, 7), (33, 252, 8), (70, 516, 9), (8, 1028, 17),
                  (100, 64, 24), (41, 300, 32)]


@pytest.mark.parametrize("dt", ["f32", "f64", "i32", "i64"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_short_k_kernel_edges(sr, dt):
    rng = np.random.default_rng(330 + tc.SEMIRINGS.index(sr))
    dtype = tc.NP_DTYPES[dt]
    for (m, n, k) in SHORTK_KERNEL_SHAPES + [(37, 132, 40), (9, 260, 63)]:
        print(f"[case] short-k {sr} {dt} m={m} n={n} k={k}", flush=True)
        a = tc.rng_matrix(rng, dtype, (m, k), -1000, 1000)
        b = tc.rng_matrix(rng, dtype, (k, n), -1000, 1000)
        ref = oracle.gemm(sr, a, b)
        c, _ = gpu_gemm(sr, a, b, False)
        assert_exact(c, None, ref[0], None)
        if k <= 32:
            assert_exact(*gpu_gemm(sr, a, b, True), *ref)


def test_short_k_kernel_integer_wrap_and_ties():
    """i32 products that wrap (MaxPlus adds near the type's limits, MaxMul
    products past 2^31) and all-equal products (argmax 0 everywhere)."""
    rng = np.random.default_rng(340)
    m, n, k = 45, 132, 12
    big = np.iinfo(np.int32).max
    a = rng.integers(big - 1000, big, size=(m, k), dtype=np.int64).astype(np.int32)
    b = rng.integers(0, 2000, size=(k, n)).astype(np.int32)
    for sr in ("maxplus", "minplus"):
        assert_exact(*gpu_gemm(sr, a, b), *oracle.gemm(sr, a, b))
    a = rng.integers(40000, 60000, size=(m, k)).astype(np.int32)
    b = rng.integers(40000, 60000, size=(k, n)).astype(np.int32)
    assert_exact(*gpu_gemm("maxmul", a, b), *oracle.gemm("maxmul", a, b))
    a = np.full((m, k), 3, np.float32)
    b = np.full((k, n), -1, np.float32)
    c, am = gpu_gemm("maxplus", a, b)
    assert np.all(c == 2) and np.all(am == 0)


@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_short_k_kernel_strided_batches(sr):
    rng = np.random.default_rng(350 + tc.SEMIRINGS.index(sr))
    m, k, n = 43, 9, 264
    items = [(tc.rng_matrix(rng, np.float32, (m, k), -100, 100),
              tc.rng_matrix(rng, np.float32, (k, n), -100, 100)) for _ in range(3)]
    for gap_a in (3, 1):
        print(f"[case] short-k strided {sr} gap_a={gap_a}", flush=True)
        out = _strided_batched(sr, items, gap_a=gap_a, gap_c=4)
        for (x, y), (c, am) in zip(items, out):
            assert_exact(c, am, *oracle.gemm(sr, x, y))


# Batches of more than 65535 products: the launches that put the batch on the
# grid's third dimension split it into chunks of 65535 items (the persistent
# K-resident kernels walk it instead).  Items on both sides of the first
# chunk boundary, and the first and last, must equal the oracle.
BIG_BATCH_CASES = [
    ("maxplus", np.float32, 4, 4, 40, True, "tiles_exact"),
    ("minplus", np.float32, 4, 4, 40, False, "shortk"),
    ("maxmul", np.float32, 3, 5, 7, False, "tiles"),
    ("maxplus", np.float32, 8, 8, 300, True, "dl_4x4_cl8"),
    ("maxplus", np.float32, 16, 12, 64, False, "dl_8x8_cl32"),
    ("minplus", np.int64, 8, 8, 300, True, "tiles_exact"),
    ("maxplus", np.float32, 64, 64, 64, True, "kres"),
]


@pytest.mark.parametrize("sr,dtype,m,n,k,with_argmax,path", BIG_BATCH_CASES,
                         ids=[f"{c[6]}-{c[0]}-{np.dtype(c[1]).name}" for c in BIG_BATCH_CASES])
def test_batch_beyond_one_grid_dimension(sr, dtype, m, n, k, with_argmax, path):
    from tropical_gemm import _native as nat

    lib = nat.load()
    batch = 65537
    dt = DT_NAME[np.dtype(dtype)]
    plan = nat.gemm_plan(sr, dt, m, n, k, with_argmax=with_argmax, batch=batch)
    print(f"[case] batch {batch} {sr} {dt} {m}x{n}x{k} argmax={with_argmax}: {plan}", flush=True)
    assert plan == path, plan
    gen = torch.Generator(device=DEV)
    gen.manual_seed(m * 1000 + k)
    tdt = TORCH_DT[np.dtype(dtype)]
    if np.dtype(dtype).kind == "f":
        ta = torch.randn(batch * m * k, generator=gen, device=DEV, dtype=tdt)
        tb = torch.randn(batch * k * n, generator=gen, device=DEV, dtype=tdt)
    else:
        ta = torch.randint(-1000, 1000, (batch * m * k,), generator=gen, device=DEV, dtype=tdt)
        tb = torch.randint(-1000, 1000, (batch * k * n,), generator=gen, device=DEV, dtype=tdt)
    c = torch.empty(batch * m * n, dtype=tdt, device=DEV)
    am = torch.empty(batch * m * n, dtype=torch.int32, device=DEV) if with_argmax else None
    nat.check(lib.tg_gemm_strided_batched(0, nat.SEMIRING[sr], nat.DTYPE[dt], 0, _p(ta), _p(tb), _p(c),
                                          _p(am), batch, m, n, k, m * k, k * n, m * n, None))
    torch.cuda.synchronize()
    for t in (0, 1, 65534, 65535, 65536):
        at = ta[t * m * k:(t + 1) * m * k].cpu().numpy().reshape(m, k)
        bt = tb[t * k * n:(t + 1) * k * n].cpu().numpy().reshape(k, n)
        ct = c[t * m * n:(t + 1) * m * n].cpu().numpy().reshape(m, n)
        c_ref, am_ref = oracle.gemm(sr, at, bt, with_argmax=with_argmax)
        if with_argmax:
            amt = am[t * m * n:(t + 1) * m * n].cpu().numpy().reshape(m, n)
            assert_exact(ct, amt, c_ref, am_ref)
        else:
            np.testing.assert_array_equal(ct, c_ref)
