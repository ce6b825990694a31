"""tg_gemm_noalloc: the forward product with the library's fixed device scratch
as its workspace, and no allocation.  Its results must equal tg_gemm's bit
for bit (values and argmax) on the same inputs.  Each case runs two calls in a
row on one device, the second with a smaller problem, so a stale scratch
from the first call would show in the second.  The rejection of a problem
whose workspace exceeds the scratch is host logic and runs without a GPU.
"""
import ctypes

import numpy as np
import pytest

from tests import tg_cases as tc
from tropical_gemm import _native as nat

SCRATCH = 64 << 20


def _lib():
    return nat.load()


def _operands(sr, dt, m, n, k, seed):
    rng = np.random.default_rng(seed)
    dtype = {"f32": np.float32, "f64": np.float64, "i32": np.int32}[dt]
    if sr == "maxmul":
        return ((1.0 - rng.random((m, k))).astype(dtype),
                (1.0 - rng.random((k, n))).astype(dtype))
    return tc.rng_matrix(rng, dtype, (m, k)), tc.rng_matrix(rng, dtype, (k, n))


def test_oversized_problem_rejected_before_device_work():
    lib = _lib()
    # argmax, 64 x 8192 x 4096 f32: B^T staging alone is 128 MiB.  Fake
    # 256-byte aligned pointers: the call must fail before dereferencing them.
    fake = ctypes.c_void_p(1 << 20)
    assert nat.gemm_plan("maxplus", "f32", 64, 8192, 4096, True,
                         workspace_bytes=SCRATCH).startswith("dl_")
    rc = lib.tg_gemm_noalloc(0, nat.SEMIRING["maxplus"], nat.DTYPE["f32"], nat.LAYOUT["row"],
                             fake, fake, fake, fake, 64, 8192, 4096, None)
    assert rc == nat.TG_ERR_INVALID_ARGUMENT
    msg = nat.last_error()
    assert "scratch" in msg and str(SCRATCH) in msg and str(4096 * 8192 * 4) in msg


def test_noalloc_bad_arguments_rejected():
    lib = _lib()
    fake = ctypes.c_void_p(1 << 20)
    rc = lib.tg_gemm_noalloc(0, 7, nat.DTYPE["f32"], nat.LAYOUT["row"], fake, fake, fake, None,
                             4, 4, 4, None)
    assert rc == nat.TG_ERR_INVALID_ARGUMENT
    rc = lib.tg_gemm_noalloc(0, nat.SEMIRING["maxplus"], nat.DTYPE["f32"], nat.LAYOUT["row"],
                             fake, fake, None, None, 4, 4, 4, None)
    assert rc == nat.TG_ERR_INVALID_ARGUMENT


# (semiring, dtype, layout, argmax, first (m, n, k), second smaller (m, n, k),
#  path of the first call with the scratch as its workspace)
CASES = [
    ("maxplus", "f32", "row", True, (2048, 2048, 2048), (256, 256, 1024), "dl_4x4_cl16"),
    ("maxplus", "f32", "row", True, (512, 512, 2048), (256, 256, 1024), "dl_4x4_cl8 split 8"),
    ("minplus", "f32", "row", True, (256, 256, 1024), (128, 192, 640), "dl_4x4_cl8 slices 4"),
    ("maxplus", "f32", "row", False, (256, 256, 1024), (128, 128, 512), "dl_4x4_cl32 split 4"),
    ("maxmul", "f64", "row", True, (64, 130, 640), (40, 64, 320), "tiles_chunked"),
    ("maxplus", "f64", "row", True, (1024, 4096, 640), (1024, 2048, 576), "dl64_4x8_cl16"),
    ("minplus", "f64", "row", False, (1024, 4096, 640), (1024, 2048, 576), "dl64_4x8"),
    ("maxplus", "i32", "col", True, (384, 256, 1024), (256, 128, 512), None),
    ("maxplus", "f32", "row", True, (3072, 4096, 1024), (512, 256, 512), "dl_4x8_cl16"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("sr,dt,layout,argmax,first,second,path", CASES,
                         ids=[f"{c[0]}-{c[1]}-{c[2]}-{'am' if c[3] else 'val'}-{c[4][0]}x{c[4][1]}x{c[4][2]}"
                              for c in CASES])
def test_noalloc_matches_tg_gemm_twice(sr, dt, layout, argmax, first, second, path):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _lib()
    dev = torch.device("cuda", 0)
    tdt = {"f32": torch.float32, "f64": torch.float64, "i32": torch.int32}[dt]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    if path is not None:
        assert nat.gemm_plan(sr, dt, *first, argmax, layout=layout, workspace_bytes=SCRATCH) == path
    for call, (m, n, k) in enumerate((first, second)):
        a, b = _operands(sr, dt, m, n, k, seed=1000 * call + m + k)
        ta = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        tb = torch.from_numpy(np.ascontiguousarray(b)).to(dev)
        outs = []
        for entry in ("tg_gemm", "tg_gemm_noalloc"):
            c = torch.full((m * n,), 7, dtype=tdt, device=dev)
            am = torch.full((m * n,), -5, dtype=torch.int32, device=dev) if argmax else None
            fn = getattr(lib, entry)
            print(f"[noalloc] call {call} {entry} {sr} {dt} {layout} {m}x{n}x{k} argmax={argmax}",
                  flush=True)
            nat.check(fn(0, nat.SEMIRING[sr], nat.DTYPE[dt], nat.LAYOUT[layout], p(ta), p(tb),
                         p(c), p(am), m, n, k, stream))
            torch.cuda.synchronize()
            outs.append((c.cpu().numpy(), am.cpu().numpy() if argmax else None))
        (c0, am0), (c1, am1) = outs
        np.testing.assert_array_equal(tc.bits(c1), tc.bits(c0))
        if argmax:
            np.testing.assert_array_equal(am1, am0)
            assert am1.min() >= 0 and am1.max() < k
