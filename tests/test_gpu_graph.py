"""The workspace entry points under HIP graph capture.

Every entry point that takes a caller workspace launches kernels only (no
allocation, no memset: buffers that must start at zero are cleared by a fill
kernel), so a caller can capture it in a HIP graph and replay it.  The test
captures the forward paths (direct-to-LDS tiles with B^T staging, 64x128
tiles, split K, the K-resident kernel, the generic tiles, their exact
short-K mode, value-only, and the f64 direct-to-LDS kernel with its operand
class prepass, with and without argmax) and both backward scatters, replays the graph
several times with new inputs copied in and eager work between the replays,
and checks every replay against eager calls on the same inputs, bit for bit
(the backward too: each gradient element receives a single contribution, so
the sum order cannot differ)."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# (name, semiring, dtype, m, k, n, argmax): one problem per forward path.
CASES = [
    ("direct-to-LDS", "maxplus", torch.float32, 2048, 1024, 2048, True),
    ("wide tiles", "minplus", torch.float32, 4096, 1024, 4096, True),
    ("split-K", "maxplus", torch.float32, 128, 4096, 128, True),
    ("K-resident", "maxplus", torch.int32, 512, 128, 128, True),
    ("generic tiles", "minplus", torch.float64, 77, 45, 93, True),
    ("exact short K", "maxplus", torch.float32, 1000, 16, 1024, True),
    ("value-only", "maxmul", torch.float32, 256, 256, 192, False),
    ("f64 direct-to-LDS", "maxplus", torch.float64, 1024, 640, 4096, True),
    ("f64 value-only", "minplus", torch.float64, 1024, 256, 4096, False),
]


def _vp(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _fill(t, gen):
    if t.dtype.is_floating_point:
        t.copy_(torch.randn(t.shape, generator=gen, device=DEV, dtype=t.dtype).abs())
    else:
        t.copy_(torch.randint(-1000, 1001, t.shape, generator=gen, device=DEV, dtype=t.dtype))


def test_forward_paths_replay_like_eager():
    from tropical_gemm import _native as nat

    lib = nat.load()
    dt_code = {torch.float32: "f32", torch.float64: "f64", torch.int32: "i32"}
    gen = torch.Generator(device=DEV)
    gen.manual_seed(77)
    bufs = []
    for name, sr, dt, m, k, n, argmax in CASES:
        a = torch.empty((m, k), dtype=dt, device=DEV)
        b = torch.empty((k, n), dtype=dt, device=DEV)
        c = torch.empty((m, n), dtype=dt, device=DEV)
        am = torch.empty((m, n), dtype=torch.int32, device=DEV) if argmax else None
        d = nat.DTYPE[dt_code[dt]]
        wsb = lib.tg_gemm_workspace_size(d, 1, m, n, k, int(argmax))
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=DEV)
        bufs.append((name, sr, d, m, k, n, a, b, c, am, ws, wsb))

    def run_all(stream):
        s = ctypes.c_void_p(stream.cuda_stream)
        for name, sr, d, m, k, n, a, b, c, am, ws, wsb in bufs:
            nat.check(lib.tg_gemm_ws(0, nat.SEMIRING[sr], d, 0, _vp(a), _vp(b), _vp(c), _vp(am),
                                     m, n, k, _vp(ws), wsb, s))

    for _, _, _, _, _, _, a, b, *_ in bufs:
        _fill(a, gen)
        _fill(b, gen)
    run_all(torch.cuda.current_stream())  # eager warm-up (device queries cached)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_all(torch.cuda.current_stream())
    for rep in range(3):
        print(f"[case] graph replay {rep}", flush=True)
        for _, _, _, _, _, _, a, b, *_ in bufs:
            _fill(a, gen)
            _fill(b, gen)
        graph.replay()
        torch.cuda.synchronize()
        got = [(c.clone(), None if am is None else am.clone()) for *_, c, am, _, _ in bufs]
        # Eager work between replays, then the eager reference on the same inputs.
        junk = torch.randn(1 << 20, device=DEV).cumsum(0)
        del junk
        run_all(torch.cuda.current_stream())
        torch.cuda.synchronize()
        for (name, *_, c, am, _, _), (gc, gam) in zip(bufs, got):
            assert torch.equal(gc.view(torch.uint8), c.view(torch.uint8)), f"{name}: values, replay {rep}"
            if am is not None:
                assert torch.equal(gam, am), f"{name}: argmax, replay {rep}"


@pytest.mark.parametrize("k", [512, 9000, 40000])
def test_backward_replays_like_eager(k):
    """grad_A and grad_B under capture: bins in LDS at K = 512 and 9000
    (grad_B in three passes over its keys at 9000), in the gradients
    themselves at K = 40000 (grad_A; grad_B takes ten passes)."""
    from tropical_gemm import _native as nat

    lib = nat.load()
    m, n = 192, 160
    gen = torch.Generator(device=DEV)
    gen.manual_seed(78)
    d = nat.DTYPE["f32"]
    g = torch.empty((m, n), device=DEV)
    # Distinct argmax per row and per column: every gradient element gets at
    # most one contribution, so results do not depend on the summation order.
    idx = torch.empty((m, n), dtype=torch.int32, device=DEV)
    ga = torch.empty((m, k), device=DEV)
    gb = torch.empty((k, n), device=DEV)

    def refill():
        g.copy_(torch.randn((m, n), generator=gen, device=DEV))
        perm = torch.randperm(k, generator=gen, device=DEV)[: m + n].to(torch.int32)
        rows = torch.arange(m, device=DEV, dtype=torch.int32)[:, None]
        cols = torch.arange(n, device=DEV, dtype=torch.int32)[None, :]
        idx.copy_(perm[(rows + cols) % (m + n)])

    def run(stream):
        s = ctypes.c_void_p(stream.cuda_stream)
        nat.check(lib.tg_backward_a(0, d, 0, _vp(g), _vp(idx), _vp(ga), m, n, k, s))
        nat.check(lib.tg_backward_b(0, d, 0, _vp(g), _vp(idx), _vp(gb), m, n, k, s))

    refill()
    run(torch.cuda.current_stream())
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(torch.cuda.current_stream())
    for rep in range(3):
        print(f"[case] backward graph replay k={k} {rep}", flush=True)
        refill()
        graph.replay()
        torch.cuda.synchronize()
        ra, rb = ga.clone(), gb.clone()
        run(torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(ra, ga) and torch.equal(rb, gb), f"replay {rep}"
        # And the scatter itself: grad_A[i, idx[i, j]] == g[i, j] (one term each).
        gh, ih = g.cpu().numpy(), idx.cpu().numpy()
        rows = np.arange(m)[:, None].repeat(n, 1)
        assert np.array_equal(ra.cpu().numpy()[rows, ih], gh)
