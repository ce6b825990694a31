"""Seeded GPU fuzz of the forward entry points against the oracle.

Random problems aimed at every dispatch path (generic tiles with ragged edges
and their exact short-K mode, direct-to-LDS full tiles, wide tiles, the
K-resident kernel with its three integer paths, split K) over all dtypes, semirings and both layouts, single
and strided-batched, with a caller workspace or the library's own.  Every
output, the gaps between strided outputs and the workspace are surrounded by
guard bytes that must come back untouched, and every result must equal the
oracle bit for bit (values as bit patterns, argmax exactly).  The backward
fuzz does the same for the gradients, which the kernels sum in the
reference's order.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from tests import tg_cases as tc

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
GUARD = 4096  # bytes before and after every output buffer and the workspace
FILL = 0x5A
NP = {"f32": np.float32, "f64": np.float64, "i32": np.int32, "i64": np.int64}
TD = {"f32": torch.float32, "f64": torch.float64, "i32": torch.int32, "i64": torch.int64}


def _p(t, byte_offset=0):
    return None if t is None else ctypes.c_void_p(t.data_ptr() + byte_offset)


def _guarded(nbytes: int) -> torch.Tensor:
    return torch.full((nbytes + 2 * GUARD,), FILL, dtype=torch.uint8, device=DEV)


def _guards_ok(buf: torch.Tensor, nbytes: int) -> bool:
    return bool(torch.all(buf[:GUARD] == FILL)) and bool(torch.all(buf[GUARD + nbytes:] == FILL))


def _shape(rng):
    kind = rng.integers(0, 7)
    if kind == 0:  # ragged, generic tiles
        return [int(x) for x in rng.integers(1, 300, size=3)], "ragged"
    if kind == 1:  # full tiles, direct-to-LDS
        return [64 * int(rng.integers(1, 6)), 32 * int(rng.integers(1, 40)),
                64 * int(rng.integers(1, 5))], "full"
    if kind == 2:  # K-resident (K in 64, 96, 128)
        return [64 * int(rng.integers(1, 8)), int(rng.choice([64, 96, 128])),
                64 * int(rng.integers(1, 4))], "kres"
    if kind == 3:  # split K: few tiles, long K
        return [64 * int(rng.integers(1, 3)), 512 * int(rng.integers(1, 9)),
                64 * int(rng.integers(1, 3))], "split"
    if kind == 5:  # short K, N % 64 == 0, any M
        return [int(rng.integers(1, 700)), int(rng.choice([32, 64, 96, 128])),
                64 * int(rng.integers(1, 6))], "short-k"
    if kind == 4:  # tiny and degenerate
        return [int(rng.integers(1, 5)), int(rng.integers(0, 40)), int(rng.integers(1, 5))], "tiny"
    return [64 * int(rng.integers(1, 4)), 32 * int(rng.integers(1, 8)),
            128 * int(rng.integers(1, 3))], "full128"


def _data(rng, dt, shape, mode, inf):
    """mode picks the distribution; inf is the one infinity used in a case
    (None: no infinities), so no product is NaN (NaN is outside the parity
    contract)."""
    if dt in ("f32", "f64"):
        if mode == 0:
            x = rng.standard_normal(shape)
        elif mode == 1:
            x = rng.integers(-3, 4, size=shape).astype(np.float64)  # many ties
        else:
            x = rng.standard_normal(shape)
            if inf is not None:
                x[rng.random(shape) < 0.1] = inf
        return x.astype(NP[dt])
    if mode == 0:
        return rng.integers(-1000, 1001, size=shape).astype(NP[dt])  # f32-key range
    if mode == 1:
        return rng.integers(-(1 << 20), 1 << 20, size=shape).astype(NP[dt])  # i32-key range
    if mode == 2:
        return rng.integers(0, 3, size=shape).astype(NP[dt])  # ties
    if mode == 4:  # f32-key range with sparse outliers: some row tiles leave the key paths
        x = rng.integers(-1000, 1001, size=shape)
        x[rng.random(shape) < 0.002] = 1 << 16
        return x.astype(NP[dt])
    info = np.iinfo(NP[dt])
    return rng.integers(info.max - 100, info.max, size=shape).astype(NP[dt])  # wraparound


@pytest.mark.parametrize("seed", range(10))
def test_forward_fuzz(seed):
    from tropical_gemm import _native as nat

    lib = nat.load()
    rng = np.random.default_rng(9000 + seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for case in range(40):
        dt = str(rng.choice(["f32", "f32", "i32", "i32", "f64", "i64"]))
        sr = str(rng.choice(tc.SEMIRINGS))
        layout = str(rng.choice(["row", "col"]))
        (m, k, n), kind = _shape(rng)
        batch = int(rng.choice([1, 1, 2, 3]))
        with_argmax = bool(rng.random() < 0.8)
        # "min": the documented minimum workspace (argmax: k x max(m, n)
        # elements per product), which leaves out the split-K partials.
        api = str(rng.choice(["ws", "alloc", "min"]))
        es = np.dtype(NP[dt]).itemsize
        # Strided batches: a gap of `gap` elements after every output matrix.
        gap = int(rng.choice([0, 0, 4, 12]))
        sc = m * n + gap
        print(f"[case] seed={seed} case={case} {kind} {sr} {dt} {layout} batch={batch} "
              f"m={m} k={k} n={n} argmax={with_argmax} api={api} gap={gap}", flush=True)
        mode = int(rng.integers(0, 5 if dt in ("i32", "i64") else 3))
        inf = None if sr == "maxmul" else (np.inf if rng.random() < 0.5 else -np.inf)
        a = [_data(rng, dt, (m, k), mode, inf) for _ in range(batch)]
        b = [_data(rng, dt, (k, n), mode, inf) for _ in range(batch)]
        if layout == "col":
            ha = np.concatenate([np.asfortranarray(x).T.ravel() for x in a])
            hb = np.concatenate([np.asfortranarray(x).T.ravel() for x in b])
        else:
            ha = np.concatenate([x.ravel() for x in a])
            hb = np.concatenate([x.ravel() for x in b])
        ta = torch.from_numpy(ha).to(DEV) if ha.size else torch.empty(1, dtype=TD[dt], device=DEV)
        tb = torch.from_numpy(hb).to(DEV) if hb.size else torch.empty(1, dtype=TD[dt], device=DEV)
        c_bytes = batch * sc * es
        i_bytes = batch * sc * 4
        cbuf = _guarded(c_bytes)
        ibuf = _guarded(i_bytes) if with_argmax else None
        ws_bytes = lib.tg_gemm_workspace_size(nat.DTYPE[dt], batch, m, n, k, int(with_argmax))
        if api == "min":
            ws_bytes = -(-(batch * k * max(m, n) * es) // 256) * 256 if with_argmax else 0
        wbuf = _guarded(ws_bytes + 256)  # room to align the workspace to 256 bytes
        woff = GUARD + (-(wbuf.data_ptr() + GUARD)) % 256
        sr_c, dt_c, lay_c = nat.SEMIRING[sr], nat.DTYPE[dt], nat.LAYOUT[layout]
        if batch == 1 and gap == 0 and rng.random() < 0.5:
            # The single-product entry points.
            if api != "alloc":
                rc = lib.tg_gemm_ws(0, sr_c, dt_c, lay_c, _p(ta), _p(tb), _p(cbuf, GUARD),
                                    _p(ibuf, GUARD) if with_argmax else None, m, n, k,
                                    _p(wbuf, woff), ws_bytes, stream)
            else:
                rc = lib.tg_gemm(0, sr_c, dt_c, lay_c, _p(ta), _p(tb), _p(cbuf, GUARD),
                                 _p(ibuf, GUARD) if with_argmax else None, m, n, k, stream)
        elif api != "alloc":
            rc = lib.tg_gemm_strided_batched_ws(
                0, sr_c, dt_c, lay_c, _p(ta), _p(tb), _p(cbuf, GUARD),
                _p(ibuf, GUARD) if with_argmax else None, batch, m, n, k, m * k, k * n, sc,
                _p(wbuf, woff), ws_bytes, stream)
        else:
            rc = lib.tg_gemm_strided_batched(
                0, sr_c, dt_c, lay_c, _p(ta), _p(tb), _p(cbuf, GUARD),
                _p(ibuf, GUARD) if with_argmax else None, batch, m, n, k, m * k, k * n, sc, stream)
        nat.check(rc)
        torch.cuda.synchronize()
        assert _guards_ok(cbuf, c_bytes), "C guard overwritten"
        if with_argmax:
            assert _guards_ok(ibuf, i_bytes), "argmax guard overwritten"
        assert bool(torch.all(wbuf[:woff] == FILL)) and bool(torch.all(wbuf[woff + ws_bytes:] == FILL)), \
            "workspace overrun"
        cv = cbuf[GUARD:GUARD + c_bytes].cpu().numpy().view(NP[dt])
        iv = ibuf[GUARD:GUARD + i_bytes].cpu().numpy().view(np.int32) if with_argmax else None
        for t in range(batch):
            c_ref, am_ref = oracle.gemm(sr, a[t], b[t], with_argmax=with_argmax)
            ct = cv[t * sc: t * sc + m * n]
            it = iv[t * sc: t * sc + m * n] if with_argmax else None
            if gap:
                assert np.all(cbuf[GUARD + (t * sc + m * n) * es: GUARD + (t + 1) * sc * es]
                              .cpu().numpy() == FILL), "gap after an output matrix overwritten"
            if layout == "col":
                ct = ct.reshape(n, m).T
                it = it.reshape(n, m).T if with_argmax else None
            else:
                ct = ct.reshape(m, n)
                it = it.reshape(m, n) if with_argmax else None
            if with_argmax:
                np.testing.assert_array_equal(tc.bits(ct), tc.bits(c_ref))
            else:
                # The sign of a value-only +-0 maximum is unpinned: compare numerically.
                np.testing.assert_array_equal(ct, c_ref)
            if with_argmax:
                np.testing.assert_array_equal(it.astype(np.int64), am_ref.astype(np.int64))


@pytest.mark.parametrize("seed", range(4))
def test_backward_fuzz(seed):
    from tropical_gemm import _native as nat

    lib = nat.load()
    rng = np.random.default_rng(9500 + seed)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for case in range(25):
        dt = str(rng.choice(["f32", "f64"]))
        m, k, n = (int(x) for x in rng.integers(1, 200, size=3))
        if rng.random() < 0.3:
            k = int(rng.choice([4096, 9000]))  # LDS-limited grad_B, and bins in global memory
        layout = str(rng.choice(["row", "col"]))
        mult = bool(rng.random() < 0.4)
        batch = int(rng.choice([1, 2]))
        which = str(rng.choice(["a", "b"]))
        print(f"[case] backward seed={seed} case={case} {dt} {layout} grad_{which} mult={mult} "
              f"batch={batch} m={m} k={k} n={n}", flush=True)
        es = np.dtype(NP[dt]).itemsize
        g = [rng.standard_normal((m, n)).astype(NP[dt]) for _ in range(batch)]
        am = [rng.integers(0, k, size=(m, n)).astype(np.int32) for _ in range(batch)]
        for x in am:
            x[rng.random(x.shape) < 0.05] = k + 3  # out of range: skipped
        other = [rng.standard_normal((k, n) if which == "a" else (m, k)).astype(NP[dt])
                 for _ in range(batch)] if mult else None

        def dev(mats):
            if layout == "col":
                h = np.concatenate([np.asfortranarray(x).T.ravel() for x in mats])
            else:
                h = np.concatenate([x.ravel() for x in mats])
            return torch.from_numpy(h).to(DEV)

        tg, tam = dev(g), dev(am)
        to = dev(other) if mult else None
        out_shape = (m, k) if which == "a" else (k, n)
        o_elems = out_shape[0] * out_shape[1]
        obuf = _guarded(batch * o_elems * es)
        s_other = (k * n if which == "a" else m * k) if mult else 0
        fn = lib.tg_backward_a_strided_batched if which == "a" else lib.tg_backward_b_strided_batched
        nat.check(fn(0, nat.DTYPE[dt], nat.LAYOUT[layout], _p(tg), _p(tam), _p(to), _p(obuf, GUARD),
                     batch, m, n, k, m * n, s_other, o_elems, stream))
        torch.cuda.synchronize()
        assert _guards_ok(obuf, batch * o_elems * es), "gradient guard overwritten"
        got = obuf[GUARD:GUARD + batch * o_elems * es].cpu().numpy().view(NP[dt])
        for t in range(batch):
            ot = got[t * o_elems:(t + 1) * o_elems]
            ot = ot.reshape(out_shape[::-1]).T if layout == "col" else ot.reshape(out_shape)
            o = other[t] if mult else None
            if which == "a":
                ref = oracle.backward_a(g[t], am[t].astype(np.uint32), k, o)
            else:
                ref = oracle.backward_b(g[t], am[t].astype(np.uint32), k, o)
            # The kernels add in the reference's order: the same bits.
            np.testing.assert_array_equal(tc.bits(np.ascontiguousarray(ot)),
                                          tc.bits(np.ascontiguousarray(ref)))


# The wide-tile paths (128 x 128 value-only, 64 x 128 value-only and argmax,
# the f64 direct-to-LDS kernel) on shapes whose last row and column tiles are
# partial, each planned onto its path (tg_gemm_plan), with guard bytes around
# C, argmax and the workspace, and sampled rows (edge tiles included) against
# the oracle.
WIDE_CASES = [
    ("maxplus", "f32", 2000, 4000, 256, False, "dl_8x8_cl32"),
    ("minplus", "i32", 2000, 4000, 256, False, "dl_8x8_cl32"),
    ("maxmul", "f32", 2000, 2048, 160, False, "dl_4x8"),
    ("maxplus", "f32", 4090, 4096, 1024, True, "dl_4x8_cl16"),
    ("minplus", "f64", 2000, 4004, 512, False, "dl64_4x8"),
    ("maxplus", "f64", 2000, 4004, 544, True, "dl64_4x8_cl16"),
]


@pytest.mark.parametrize("sr,dt,m,n,k,with_argmax,path", WIDE_CASES,
                         ids=[f"{c[6]}-{c[0]}-{c[1]}-{c[2]}x{c[3]}x{c[4]}" for c in WIDE_CASES])
def test_wide_paths_guarded(sr, dt, m, n, k, with_argmax, path):
    from tropical_gemm import _native as nat

    lib = nat.load()
    assert nat.gemm_plan(sr, dt, m, n, k, with_argmax) == path
    print(f"[case] guarded {path} {sr} {dt} {m}x{n}x{k} argmax={with_argmax}", flush=True)
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    if dt in ("f32", "f64"):
        a = rng.standard_normal((m, k)).astype(NP[dt])
        b = rng.standard_normal((k, n)).astype(NP[dt])
        if sr == "maxmul":
            a, b = np.abs(a), np.abs(b)
    else:
        a = rng.integers(-1000, 1001, size=(m, k)).astype(NP[dt])
        b = rng.integers(-1000, 1001, size=(k, n)).astype(NP[dt])
    es = np.dtype(NP[dt]).itemsize
    ta, tb = torch.from_numpy(a).to(DEV), torch.from_numpy(b).to(DEV)
    c_bytes, i_bytes = m * n * es, m * n * 4
    cbuf = _guarded(c_bytes)
    ibuf = _guarded(i_bytes) if with_argmax else None
    ws_bytes = lib.tg_gemm_workspace_size(nat.DTYPE[dt], 1, m, n, k, int(with_argmax))
    wbuf = _guarded(ws_bytes + 256)
    woff = GUARD + (-(wbuf.data_ptr() + GUARD)) % 256
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.check(lib.tg_gemm_ws(0, nat.SEMIRING[sr], nat.DTYPE[dt], nat.LAYOUT["row"], _p(ta), _p(tb),
                             _p(cbuf, GUARD), _p(ibuf, GUARD) if with_argmax else None, m, n, k,
                             _p(wbuf, woff), ws_bytes, stream))
    torch.cuda.synchronize()
    assert _guards_ok(cbuf, c_bytes), "C guard overwritten"
    if with_argmax:
        assert _guards_ok(ibuf, i_bytes), "argmax guard overwritten"
    assert bool(torch.all(wbuf[:woff] == FILL)) and bool(torch.all(wbuf[woff + ws_bytes:] == FILL)), \
        "workspace overrun"
    c = cbuf[GUARD:GUARD + c_bytes].cpu().numpy().view(NP[dt]).reshape(m, n)
    rows = np.unique(np.concatenate([np.arange(0, m, 97), [63, 64, 127, 128, m - 2, m - 1]]))
    c_ref, am_ref = oracle.gemm(sr, a[rows], b, with_argmax=with_argmax)
    if with_argmax:
        am = ibuf[GUARD:GUARD + i_bytes].cpu().numpy().view(np.int32).reshape(m, n)
        np.testing.assert_array_equal(tc.bits(c[rows]), tc.bits(c_ref))
        np.testing.assert_array_equal(am[rows].astype(np.int64), am_ref.astype(np.int64))
    else:
        np.testing.assert_array_equal(c[rows], c_ref)
