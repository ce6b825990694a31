"""Tropical einsum on the CPU: the brute-force oracle pinned against the GEMM
oracle and closed forms, and the host-side logic of the einsum engine
(parsing, index classes, contraction order)."""
import math

import numpy as np
import pytest

from oracle import einsum_ref as er
from oracle import oracle
from tests import tg_cases as tc


@pytest.mark.parametrize("dt", ["f32", "i32"])
@pytest.mark.parametrize("sr", tc.SEMIRINGS)
def test_binary_ref_matrix_product_equals_gemm_oracle(sr, dt):
    rng = np.random.default_rng(7)
    dtype = tc.NP_DTYPES[dt]
    lo = 0 if sr == "maxmul" else -5
    a = tc.rng_matrix(rng, dtype, (5, 7), lo, 5)
    b = tc.rng_matrix(rng, dtype, (7, 4), lo, 5)
    y, idx = er.contract_binary_ref(a, b, "ij", "jk", "ik", sr)
    c, am = oracle.gemm(sr, a, b)
    np.testing.assert_array_equal(tc.bits(y), tc.bits(c))
    np.testing.assert_array_equal(idx, am.astype(np.int64))
    # Output order is a permutation of the same values.
    yt, it = er.contract_binary_ref(a, b, "ij", "jk", "ki", sr)
    np.testing.assert_array_equal(tc.bits(yt), tc.bits(c.T))
    np.testing.assert_array_equal(it, am.T.astype(np.int64))


def test_binary_ref_closed_forms():
    rng = np.random.default_rng(8)
    a = rng.integers(-9, 10, size=6).astype(np.int32)
    b = rng.integers(-9, 10, size=6).astype(np.int32)
    y, idx = er.contract_binary_ref(a, b, "i", "i", "", "maxplus")  # dot
    assert y == (a + b).max() and idx == int(np.argmax(a + b))
    y, _ = er.contract_binary_ref(a, b, "i", "i", "", "minplus")
    assert y == (a + b).min()
    y, idx = er.contract_binary_ref(a, b, "i", "j", "ij", "maxplus")  # outer product
    np.testing.assert_array_equal(y, a[:, None] + b[None, :])
    assert np.all(idx == 0)
    # A label summed in one operand only: (max_j A[i,j]) + B[i].
    m = rng.integers(-9, 10, size=(6, 4)).astype(np.int32)
    y, idx = er.contract_binary_ref(m, b, "ij", "i", "i", "maxplus")
    np.testing.assert_array_equal(y, m.max(axis=1) + b)
    assert idx is None
    # Batch label: the k-th diagonal block products.
    p = rng.integers(-9, 10, size=(3, 4, 5)).astype(np.int32)
    q = rng.integers(-9, 10, size=(3, 5, 2)).astype(np.int32)
    y, idx = er.contract_binary_ref(p, q, "bij", "bjk", "bik", "maxplus")
    for t in range(3):
        c, am = oracle.gemm("maxplus", p[t], q[t])
        np.testing.assert_array_equal(y[t], c)
        np.testing.assert_array_equal(idx[t], am)


def test_einsum_ref_closed_forms():
    rng = np.random.default_rng(9)
    m = rng.integers(-9, 10, size=(5, 5)).astype(np.int64)
    assert er.einsum_ref(["ii"], "", [m], "maxplus") == np.diag(m).max()  # tropical trace
    assert er.einsum_ref(["ij"], "", [m], "minplus") == m.min()
    np.testing.assert_array_equal(er.einsum_ref(["ij"], "ji", [m], "maxplus"), m.T)
    np.testing.assert_array_equal(er.einsum_ref(["ii"], "i", [m], "maxplus"), np.diag(m))
    # Chain of three = two GEMMs (integer data: association does not matter).
    a = rng.integers(-9, 10, size=(3, 4)).astype(np.int32)
    b = rng.integers(-9, 10, size=(4, 5)).astype(np.int32)
    c = rng.integers(-9, 10, size=(5, 2)).astype(np.int32)
    ab, _ = oracle.gemm("maxplus", a, b)
    abc, _ = oracle.gemm("maxplus", ab, c)
    np.testing.assert_array_equal(er.einsum_ref(["ij", "jk", "kl"], "il", [a, b, c], "maxplus"), abc)


def test_binary_ref_rejects_a_planted_mistake(monkeypatch):
    """With the strict-improvement rule replaced by >= (last maximum wins),
    the restatement must disagree with the GEMM oracle on ties: the check
    above is able to catch that mistake."""
    a = np.zeros((2, 4), np.int32)
    b = np.zeros((4, 3), np.int32)
    _, am = oracle.gemm("maxplus", a, b)
    _, idx = er.contract_binary_ref(a, b, "ij", "jk", "ik", "maxplus")
    np.testing.assert_array_equal(idx, am.astype(np.int64))
    monkeypatch.setattr(er, "_better", lambda sr, cand, acc: cand >= acc)
    _, idx_bad = er.contract_binary_ref(a, b, "ij", "jk", "ik", "maxplus")
    assert not np.array_equal(idx_bad, am.astype(np.int64))


def test_parse_and_classify():
    from tropical_gemm import einsum as E

    assert E.parse("ij,jk->ik") == ([["i", "j"], ["j", "k"]], ["i", "k"])
    assert E.parse("ij, jk") == ([["i", "j"], ["j", "k"]], ["i", "k"])  # implicit output
    assert E.parse("ii") == ([["i", "i"]], [])
    with pytest.raises(ValueError, match="ellipsis"):
        E.parse("...ij,jk->ik")
    with pytest.raises(ValueError, match="operands"):
        E.parse("ij,jk->ik", 3)
    with pytest.raises(ValueError, match="invalid label"):
        E.parse("i1,jk->ik")
    cls = E.classify(list("bijx"), list("bjky"), list("bki"))
    assert cls == {"batch": ["b"], "left": ["i"], "right": ["k"], "contracted": ["j"],
                   "a_sum": ["x"], "b_sum": ["y"]}
    with pytest.raises(ValueError, match="neither operand"):
        E.classify(list("ij"), list("jk"), list("iz"))
    with pytest.raises(ValueError, match="repeat"):
        E.classify(list("ij"), list("jk"), list("ii"))


def test_contraction_order():
    from tropical_gemm import einsum as E

    ixs = [list("ij"), list("jk"), list("kl")]
    # Small l: contract the right pair first (intermediate j x l).
    assert E.einsum_path(ixs, list("il"), {"i": 100, "j": 100, "k": 100, "l": 2}) == [(1, 2), (0, 1)]
    # Small i: the left pair first.
    assert E.einsum_path(ixs, list("il"), {"i": 2, "j": 100, "k": 100, "l": 100}) == [(0, 1), (0, 1)]
    # optimize=None: left to right whatever the sizes.
    assert E.einsum_path(ixs, list("il"), {"i": 100, "j": 100, "k": 100, "l": 2}, None) == [(0, 1), (0, 1)]
    # A ring a-b-c-d-a: every step keeps the labels still shared with the rest.
    ring = [list("ab"), list("bc"), list("cd"), list("da")]
    path = E.einsum_path(ring, [], {x: 3 for x in "abcd"})
    assert len(path) == 3
    with pytest.raises(ValueError, match="optimize"):
        E.einsum_path(ixs, list("il"), {x: 2 for x in "ijkl"}, "dp")


def test_layout_copies_route_group_swaps_to_the_transpose(monkeypatch):
    """The einsum's operand copies: a permutation that moves one group of
    adjacent axes past another goes to ``ops.transpose`` as a (batched) 2-D
    transpose, any other to torch, and either way the result equals
    ``permute(perm).contiguous()`` (host logic, with the device transpose
    replaced by torch's)."""
    import itertools

    torch = pytest.importorskip("torch")
    from tropical_gemm import einsum as E, ops

    calls = []

    def fake_transpose(x):
        calls.append(tuple(x.shape))
        return x.transpose(-1, -2).contiguous()

    monkeypatch.setattr(ops, "transpose", fake_transpose)
    monkeypatch.setattr(E, "_needs_grad", lambda *ts: False)
    n = 0
    for shape in [(2, 3, 4), (5, 1, 3, 2), (2, 3, 4, 5), (1, 4, 1, 3), (3, 1, 1, 2, 4)]:
        t = torch.arange(math.prod(shape), dtype=torch.float32).reshape(shape)
        for perm in itertools.permutations(range(len(shape))):
            got = E._layout(t, list(perm))
            ref = t.permute(perm).contiguous()
            assert got.is_contiguous() and got.shape == ref.shape and torch.equal(got, ref), (shape, perm)
            n += 1
    assert n == 198 and len(calls) == 93
    # [j, i, k] -> [k, j, i] is one transpose of a (j i) x k matrix.
    calls.clear()
    E._layout(torch.zeros(32, 64, 16), [2, 0, 1])
    assert calls == [(32 * 64, 16)]
    # [z, a, b] -> [z, b, a]: a batch of transposes.
    calls.clear()
    E._layout(torch.zeros(3, 5, 7), [0, 2, 1])
    assert calls == [(3, 5, 7)]
