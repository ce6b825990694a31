"""C ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching the device."""
import ctypes
import os
import re

import pytest

from tropical_gemm import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tropical_gemm_hip.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tg_[a-z0-9_]+)\s*\(", text)))


def test_library_built():
    assert os.path.exists(nat.library_path()), "run __graft_entry__.build() first"


def test_every_declared_symbol_is_exported_and_bound():
    lib = nat.load()
    declared = header_symbols()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(nat.SIGNATURES) == declared, "ctypes signatures out of sync with the header"


def test_version_and_status_strings():
    lib = nat.load()
    assert lib.tg_version() == 1
    assert lib.tg_status_string(nat.TG_ERR_DIMENSION_MISMATCH) == b"dimension mismatch"
    assert lib.tg_status_string(999) == b"unknown status"


def _gemm(**kw):
    args = dict(device=0, sr=0, dt=0, layout=0, A=1, B=1, C=1, argmax=None, m=4, n=4, k=4)
    args.update(kw)
    lib = nat.load()
    p = lambda v: None if v is None else ctypes.c_void_p(v)  # noqa: E731
    return lib.tg_gemm(args["device"], args["sr"], args["dt"], args["layout"], p(args["A"]),
                       p(args["B"]), p(args["C"]), p(args["argmax"]), args["m"], args["n"],
                       args["k"], None)


@pytest.mark.parametrize("kw,status,needle", [
    (dict(sr=7), nat.TG_ERR_INVALID_ARGUMENT, "unknown semiring"),
    (dict(dt=9), nat.TG_ERR_INVALID_ARGUMENT, "unknown dtype"),
    (dict(layout=3), nat.TG_ERR_INVALID_ARGUMENT, "unknown layout"),
    (dict(m=-1), nat.TG_ERR_DIMENSION_MISMATCH, "negative dimension"),
    (dict(k=2**31), nat.TG_ERR_DIMENSION_MISMATCH, "2^31-1"),
    (dict(C=None), nat.TG_ERR_INVALID_ARGUMENT, "C is NULL"),
    (dict(A=None), nat.TG_ERR_INVALID_ARGUMENT, "A or B is NULL"),
])
def test_gemm_argument_validation(kw, status, needle):
    assert _gemm(**kw) == status
    assert needle in nat.last_error()


def test_workspace_size_and_validation():
    lib = nat.load()
    assert lib.tg_gemm_workspace_size(0, 1, 64, 64, 64, 0) == 0
    need = lib.tg_gemm_workspace_size(0, 1, 100, 70, 33, 1)
    # B^T staging covers the wider of m and n: column-major calls swap the
    # operands, so the kernel's B is A (k x m).
    assert need >= 100 * 33 * 4 and need % 256 == 0
    assert lib.tg_gemm_workspace_size(0, 1, 70, 100, 33, 1) == need
    assert lib.tg_gemm_workspace_size(1, 2, 10, 10, 10, 1) >= 2 * 10 * 10 * 8
    rc = lib.tg_gemm_ws(0, 0, 0, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                        ctypes.c_void_p(16), 8, 8, 8, ctypes.c_void_p(256), 16, None)
    assert rc == nat.TG_ERR_INVALID_ARGUMENT and "workspace too small" in nat.last_error()


def test_batched_output_overlap_rejected():
    lib = nat.load()
    p = ctypes.c_void_p(4096)
    rc = lib.tg_gemm_strided_batched(0, 0, 0, 0, p, p, p, None, 3, 4, 4, 4, 16, 16, 8, None)
    assert rc == nat.TG_ERR_DIMENSION_MISMATCH and "overlap" in nat.last_error()


def test_backward_rejects_integer_dtype():
    lib = nat.load()
    p = ctypes.c_void_p(4096)
    rc = lib.tg_backward_a(0, nat.DTYPE["i32"], 0, p, p, p, 4, 4, 4, None)
    assert rc == nat.TG_ERR_UNSUPPORTED and "f32/f64" in nat.last_error()


def test_maxmul_backward_needs_operand():
    lib = nat.load()
    p = ctypes.c_void_p(4096)
    rc = lib.tg_maxmul_backward_a(0, 0, 0, p, p, None, p, 4, 4, 4, None)
    assert rc == nat.TG_ERR_INVALID_ARGUMENT and "other operand" in nat.last_error()


def test_hip_error_maps_reference_variants():
    e = nat.HipError(nat.TG_ERR_DIMENSION_MISMATCH, "A.cols (3) != B.rows (4)")
    assert e.kind == "DimensionMismatch" and "A.cols" in str(e)
    assert nat.HipError(nat.TG_ERR_NO_DEVICE, "x").kind == "NoDevice"


def test_python_layer_rejects_host_tensors():
    torch = pytest.importorskip("torch")
    from tropical_gemm import ops

    a = torch.zeros(2, 3)
    b = torch.zeros(3, 2)
    with pytest.raises(ValueError, match="device tensors"):
        ops.gemm("maxplus", a, b)
    with pytest.raises(ValueError, match="Expected 2D"):
        ops.gemm("maxplus", a, torch.zeros(3))
    with pytest.raises(ValueError, match="same dtype"):
        ops.gemm("maxplus", a, torch.zeros(3, 2, dtype=torch.float64))


# ---------------------------------------------------------------------------
# Dispatch and launch geometry (host logic; no device needed)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("sr,dt,m,n,k,argmax,expected", [
    ("maxplus", "f32", 4096, 4096, 4096, True, "dl_4x8_cl16"),       # P
    ("minplus", "f32", 4096, 4096, 4096, True, "dl_4x8_cl16"),       # C2
    ("maxmul", "f32", 8192, 4096, 2048, False, "dl_8x8_cl32"),       # C3
    ("maxplus", "i32", 262144, 128, 128, True, "kresw"),             # C4
    ("maxplus", "f32", 1024, 1024, 1024, True, "dl_4x4_cl8 slices 4"),  # C1
    ("maxplus", "f32", 65536, 8, 2048, True, "shortk"),              # M1 (m, k, n order below)
    ("maxplus", "f32", 67, 45, 40, True, "tiles_exact"),
    ("maxplus", "f64", 4096, 4096, 4096, True, "dl64_4x8_cl16"),
    ("maxplus", "f64", 64, 64, 640, True, "tiles_chunked"),
    ("maxplus", "f64", 4096, 4096, 4096, False, "dl64_4x8"),
    ("maxplus", "f64", 4096, 4096, 128, False, "tiles"),
    ("maxplus", "f32", 2048, 2048, 2048, False, "dl_4x8"),           # E1's GEMMs: one 64x64 round
    ("minplus", "f32", 2048, 4096, 1024, False, "dl_8x8_cl32"),      # one 128x128 round
    ("maxplus", "f32", 3072, 3072, 2048, False, "dl_4x4_cl32"),      # 1.125 rounds of 128x128
    ("maxplus", "f32", 1536, 2048, 2048, False, "dl_4x4_cl32"),      # 0.75 rounds of 64x64
])
def test_gemm_plan_names_the_configured_paths(sr, dt, m, n, k, argmax, expected):
    if expected == "shortk":
        m, n, k = 65536, 2048, 8
    assert nat.gemm_plan(sr, dt, m, n, k, argmax) == expected


def test_gemm_plan_rejects_what_the_call_rejects():
    assert nat.gemm_plan("maxplus", "f32", -1, 4, 4) == "invalid"
    assert nat.gemm_plan("maxplus", "f32", 0, 4, 4) == "none"


@pytest.mark.parametrize("dt", [0, 1])
@pytest.mark.parametrize("want_a", [1, 0])
@pytest.mark.parametrize("shape", [(1, 4096, 4096, 4096), (1, (1 << 24) + 1, 2, 3),
                                   (1, 3, (1 << 31) - 1, 3), (65535 * 4, 64, 64, 64),
                                   (1, 5, 9000, 100000), (3, 2, 2, 1 << 30)])
def test_backward_geometry_caps_every_launch_dimension(dt, want_a, shape):
    """Grid-stride kernels: whatever M, N, K and batch, the grid stays at or
    below 16384 workgroups of at most 512 threads, and LDS within the CU."""
    batch, m, n, k = shape
    lib = nat.load()
    for layout in (0, 1):
        plan = lib.tg_backward_plan(dt, layout, want_a, batch, m, n, k).decode()
        fields = dict(f.split("=") for f in plan.split()[2:])
        assert 1 <= int(fields["grid"]) <= 16384, plan
        assert 1 <= int(fields["waves"]) <= 8, plan
        assert int(fields["lds"]) <= 160 * 1024, plan
        elem = 4 if dt == 0 else 8
        if k * elem > 128 * 1024:
            assert "global" in plan, plan


def _noalloc_bytes(sr, dt, m, n, k, argmax, layout="row"):
    lib = nat.load()
    return lib.tg_gemm_noalloc_bytes(nat.SEMIRING[sr], nat.DTYPE[dt], nat.LAYOUT[layout], 256, 256,
                                     256, 256 if argmax else None, m, n, k)


def _round256(x):
    return -(-x // 256) * 256


@pytest.mark.parametrize("m,n,k,argmax", [(2048, 2048, 1024, True), (2048, 2048, 1024, False),
                                          (1024, 2048, 512, False), (2000, 4004, 544, True)])
def test_noalloc_bytes_cover_the_f64_direct_to_lds_workspace(m, n, k, argmax):
    """f64 problems on the direct-to-LDS kernel read B^T (argmax) and the
    operand classes (4 bytes per row of A and per column of B) from the
    workspace: tg_gemm_noalloc's scratch need counts both."""
    plan = nat.gemm_plan("maxplus", "f64", m, n, k, argmax, workspace_bytes=64 << 20)
    assert plan.startswith("dl64"), plan
    want = (_round256(k * n * 8) if argmax else 0) + _round256((m + n) * 4)
    assert _noalloc_bytes("maxplus", "f64", m, n, k, argmax) == want


def test_noalloc_bytes_of_other_paths():
    # 32-bit argmax on the direct-to-LDS kernel: B^T staging (row-major: k x n).
    assert nat.gemm_plan("maxplus", "f32", 4096, 4096, 4096, True) == "dl_4x8_cl16"
    assert _noalloc_bytes("maxplus", "f32", 4096, 4096, 4096, True) == 4096 * 4096 * 4
    # Split K: the value and index partials after the (here unused) B^T region.
    assert nat.gemm_plan("maxplus", "f32", 1024, 1024, 1024, True,
                         workspace_bytes=64 << 20) == "dl_4x4_cl8 slices 4"
    assert _noalloc_bytes("maxplus", "f32", 1024, 1024, 1024, True) == \
        1024 * 1024 * 4 + 2 * (2 * 1024 * 1024 * 4)
    # Paths without workspace, and empty products.
    assert _noalloc_bytes("maxplus", "f32", 4096, 4096, 4096, False) == 0
    assert _noalloc_bytes("maxplus", "i32", 262144, 128, 128, True) == 0
    assert _noalloc_bytes("maxplus", "f32", 0, 4, 4, True) == 0
    assert _noalloc_bytes("maxplus", "f32", -1, 4, 4, True) == 2**64 - 1
