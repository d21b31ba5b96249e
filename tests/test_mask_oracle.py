"""CPU pins of the mask oracle: numpy.packbits's bit order against an
element-by-element restatement, segment offsets, and the tree mask against
closed forms (a plausible slip -- wrong bit order, a missing prefix column,
Anc transposed -- fails one of these)."""
import numpy as np
import pytest

from oracle import gdn_tree as O
from oracle import mask as M

RNG = np.random.default_rng(77)


@pytest.mark.parametrize("bitorder", ["little", "big"])
def test_packbits_matches_loop(bitorder):
    for n in list(range(0, 41)) + [255, 256, 257, 1000]:
        x = RNG.integers(0, 3, size=n).astype(np.uint8)  # values 2 count as 1
        assert np.array_equal(M.packbits(x, bitorder), M.packbits_loop(x, bitorder)), n


def test_packbits_little_known_bytes():
    # element 0 is the lowest bit of byte 0; padding bits are zero
    assert M.packbits([1, 0, 0, 0, 0, 0, 0, 0]).tolist() == [1]
    assert M.packbits([0, 0, 0, 0, 0, 0, 0, 1]).tolist() == [128]
    assert M.packbits([1] * 9).tolist() == [255, 1]
    assert M.packbits([1, 0, 0, 0, 0, 0, 0, 0], "big").tolist() == [128]


def test_segment_packbits_offsets():
    x = RNG.integers(0, 2, size=100).astype(bool)
    indptr = [0, 0, 9, 17, 17, 64, 100]
    packed, new = M.segment_packbits(x, indptr)
    lens = np.diff(indptr)
    assert new.tolist() == np.concatenate([[0], np.cumsum((lens + 7) // 8)]).tolist()
    for s in range(len(lens)):
        assert np.array_equal(packed[new[s]:new[s + 1]], M.packbits_loop(x[indptr[s]:indptr[s + 1]]))


def _parent(n, kind):
    p = np.full(n, -1, np.int64)
    for i in range(1, n):
        p[i] = i - 1 if kind == "chain" else (0 if kind == "bushy" else RNG.integers(0, i))
    return p


@pytest.mark.parametrize("plen", [0, 1, 5, 8, 33])
def test_tree_mask_closed_forms(plen):
    n = 12
    anc, _, _ = O.tree_struct(_parent(n, "chain"))
    m = M.tree_mask(anc, plen)
    assert m.shape == (n, plen + n)
    assert m[:, :plen].all()
    assert np.array_equal(m[:, plen:], np.tril(np.ones((n, n), bool)))  # a chain: every earlier node
    anc, _, _ = O.tree_struct(_parent(n, "bushy"))
    m = M.tree_mask(anc, plen)
    assert np.array_equal(m[:, plen:], np.eye(n, dtype=bool) | (np.arange(n)[None, :] == 0))  # self and the root
    parent = _parent(n, "random")
    anc, _, _ = O.tree_struct(parent)
    m = M.tree_mask(anc, plen)
    for i in range(n):
        walk = {i}
        j = i
        while j != 0:
            j = int(parent[j])
            walk.add(j)
        assert set(np.flatnonzero(m[i, plen:]).tolist()) == walk
    # the packed form is the row-major flattening, rows not byte-aligned
    assert np.array_equal(M.tree_mask_packed(anc, plen), M.packbits_loop(m.reshape(-1)))
