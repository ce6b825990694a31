"""Seeded synthetic inputs for the benchmark configurations.

Inputs are generated on the device with torch's Philox generator from fixed
seeds, so a run feeds the same tensors to the GPU kernels and (after a copy to
the host) to the CPU oracle.  Nothing here reads the reference.

    P   MaxPlus f32 4096^3 with argmax, A, B ~ N(0,1)           (headline)
    C1  MaxPlus f32 1024^3, value-only and with argmax, N(0,1)
    C2  MinPlus f32 4096^3 with argmax; U[0,100), 10% +inf, zero diagonal
    C3  MaxMul f32 value-only, M=8192 K=2048 N=4096, entries in (0,1]
    C4  MaxPlus i32 M=262144 K=128 N=128 with argmax; A in [-1000,1000], B in [-50,0]
    C5  P forward, then backward with dC ~ N(0,1)
    M1  MaxPlus f32 M=65536 K=8 N=2048 with argmax, N(0,1): short K, bound by
        HBM (the 0.5 GB output and argmax writes), not by the VALU
    F1  MaxPlus f64 4096^3 with argmax, A, B ~ N(0,1) (the f64 kernels)
    F2  MaxPlus f64 4096^3 value-only, A, B ~ N(0,1)
    I1  MaxPlus i64 4096^3 with argmax, A, B uniform integers in [-10^9, 10^9]
    I2  MaxPlus i64 4096^3 value-only, same inputs
    E1  tropical einsum "jik,lkj,lm->im", MaxPlus f32, N(0,1): i = l = m = 2048,
        j = 32, k = 64 (two 2048^3 contractions after two permutations)
"""
from __future__ import annotations

import torch

SEED_BASE = 0x7E0000

CONFIGS = {
    "P": dict(semiring="maxplus", dtype="f32", m=4096, k=4096, n=4096, argmax=True),
    "C1": dict(semiring="maxplus", dtype="f32", m=1024, k=1024, n=1024, argmax=True),
    "C2": dict(semiring="minplus", dtype="f32", m=4096, k=4096, n=4096, argmax=True),
    "C3": dict(semiring="maxmul", dtype="f32", m=8192, k=2048, n=4096, argmax=False),
    "C4": dict(semiring="maxplus", dtype="i32", m=262144, k=128, n=128, argmax=True),
    "C5": dict(semiring="maxplus", dtype="f32", m=4096, k=4096, n=4096, argmax=True,
               backward=True),
    "M1": dict(semiring="maxplus", dtype="f32", m=65536, k=8, n=2048, argmax=True, bound="hbm"),
    "F1": dict(semiring="maxplus", dtype="f64", m=4096, k=4096, n=4096, argmax=True),
    "F2": dict(semiring="maxplus", dtype="f64", m=4096, k=4096, n=4096, argmax=False),
    "I1": dict(semiring="maxplus", dtype="i64", m=4096, k=4096, n=4096, argmax=True),
    "I2": dict(semiring="maxplus", dtype="i64", m=4096, k=4096, n=4096, argmax=False),
}


def _gen(device, config_idx: int, tensor_id: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(SEED_BASE + 16 * config_idx + tensor_id)
    return g


def make_inputs(name: str, device="cuda", scale: float = 1.0):
    """Return (A, B) for config `name`; `scale` < 1 shrinks M (and N, K for the
    square configs) for quick parity runs with the same distributions."""
    cfg = CONFIGS[name]
    idx = list(CONFIGS).index(name)
    m = max(1, int(cfg["m"] * scale))
    k = cfg["k"] if name == "C4" else max(1, int(cfg["k"] * scale))
    n = cfg["n"] if name == "C4" else max(1, int(cfg["n"] * scale))
    if name in ("P", "C1", "C5", "M1", "F1", "F2"):
        dt = torch.float64 if cfg["dtype"] == "f64" else torch.float32
        a = torch.randn(m, k, generator=_gen(device, idx, 0), device=device, dtype=dt)
        b = torch.randn(k, n, generator=_gen(device, idx, 1), device=device, dtype=dt)
    elif name == "C2":
        a = _distance_matrix(m, k, device, _gen(device, idx, 0), _gen(device, idx, 3))
        b = _distance_matrix(k, n, device, _gen(device, idx, 1), _gen(device, idx, 4))
    elif name == "C3":
        a = 1.0 - torch.rand(m, k, generator=_gen(device, idx, 0), device=device)
        b = 1.0 - torch.rand(k, n, generator=_gen(device, idx, 1), device=device)
    elif name == "C4":
        a = torch.randint(-1000, 1001, (m, k), generator=_gen(device, idx, 0), device=device,
                          dtype=torch.int32)
        b = torch.randint(-50, 1, (k, n), generator=_gen(device, idx, 1), device=device,
                          dtype=torch.int32)
    elif name in ("I1", "I2"):
        lim = 10**9
        a = torch.randint(-lim, lim + 1, (m, k), generator=_gen(device, idx, 0), device=device,
                          dtype=torch.int64)
        b = torch.randint(-lim, lim + 1, (k, n), generator=_gen(device, idx, 1), device=device,
                          dtype=torch.int64)
    else:
        raise KeyError(name)
    return a.contiguous(), b.contiguous()


def _distance_matrix(r, c, device, g_val, g_mask):
    d = torch.rand(r, c, generator=g_val, device=device, dtype=torch.float64) * 100.0
    d = d.to(torch.float32).clamp_(max=float(torch.nextafter(torch.tensor(100.0),
                                                             torch.tensor(0.0))))
    mask = torch.rand(r, c, generator=g_mask, device=device) < 0.10
    d[mask] = float("inf")
    diag = min(r, c)
    idx = torch.arange(diag, device=device)
    d[idx, idx] = 0.0
    return d


EINSUM = {
    "E1": dict(code="jik,lkj,lm->im", semiring="maxplus", dtype="f32",
               sizes=dict(i=2048, j=32, k=64, l=2048, m=2048)),
}


def make_einsum_operands(name: str, device="cuda"):
    """Operands of einsum workload `name` (seeded like the GEMM configs)."""
    cfg = EINSUM[name]
    idx = len(CONFIGS) + list(EINSUM).index(name)
    lhs = cfg["code"].split("->")[0].split(",")
    return [torch.randn([cfg["sizes"][x] for x in term], generator=_gen(device, idx, t),
                        device=device) for t, term in enumerate(lhs)]


def make_grad(name: str, m: int, n: int, device="cuda", dtype=torch.float32):
    idx = list(CONFIGS).index(name)
    return torch.randn(m, n, generator=_gen(device, idx, 2), device=device, dtype=dtype)
