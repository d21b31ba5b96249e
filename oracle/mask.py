"""CPU oracle for the bit-packed attention masks.

TEST INFRASTRUCTURE ONLY (see the package docstring): the reference that
the tests hold ``dft_packbits`` and ``dft_tree_mask_pack`` against, never
called by the product.

* ``packbits`` / ``segment_packbits``   flashinfer.packbits / segment_packbits
  as fc1_plan.py:26 calls them: numpy.packbits (the library routine) per
  segment, segment s starting at byte sum_{s'<s} ceil(len_s' / 8).
* ``tree_mask``                          the boolean mask of fc1_branch64.py:39:
  [ones(n, plen) | Anc] row-major (Anc = ancestor-or-self, as tree_struct).
* ``tree_mask_packed``                   its packed form (fc1_plan.py:26).
* ``packbits_loop``                      element-by-element restatement of the
  bit order, used to pin numpy.packbits's reading of "little" / "big".

Pinning: ``packbits`` is numpy.packbits itself; tests/test_mask_oracle.py
checks it against ``packbits_loop`` (lengths 0-40 and random), and checks
``tree_mask`` against closed forms (a chain gives a lower-triangular tree part,
every row's prefix is all ones, row i's tree part is its ancestor set from the
parent walk).
"""
from __future__ import annotations

import numpy as np


def packbits(x, bitorder: str = "little") -> np.ndarray:
    """numpy.packbits of the flattened x, any non-zero element counting as 1."""
    return np.packbits(np.asarray(x).reshape(-1) != 0, bitorder=bitorder)


def packbits_loop(x, bitorder: str = "little") -> np.ndarray:
    """Element 8j + k is bit k (little) or bit 7 - k (big) of byte j."""
    x = [1 if v else 0 for v in np.asarray(x).reshape(-1).tolist()]
    out = np.zeros((len(x) + 7) // 8, dtype=np.uint8)
    for e, v in enumerate(x):
        j, k = divmod(e, 8)
        if v:
            out[j] |= np.uint8(1 << (k if bitorder == "little" else 7 - k))
    return out


def segment_packbits(x, indptr, bitorder: str = "little"):
    """(packed bytes of every segment back to back, new indptr in bytes)."""
    x = np.asarray(x).reshape(-1)
    indptr = np.asarray(indptr, dtype=np.int64)
    parts, new = [], [0]
    for s in range(len(indptr) - 1):
        lo, hi = int(indptr[s]), int(indptr[s + 1])
        p = packbits(x[lo:max(hi, lo)], bitorder)
        parts.append(p)
        new.append(new[-1] + p.size)
    packed = np.concatenate(parts) if parts else np.zeros(0, dtype=np.uint8)
    return packed, np.asarray(new, dtype=np.int64)


def tree_mask(anc, plen: int) -> np.ndarray:
    """fc1_branch64.py:39: torch.cat((ones(n, plen), anc.bool()), dim=1)."""
    anc = np.asarray(anc) > 0.5
    n = anc.shape[0]
    return np.concatenate([np.ones((n, plen), dtype=bool), anc], axis=1)


def tree_mask_packed(anc, plen: int, bitorder: str = "little") -> np.ndarray:
    return packbits(tree_mask(anc, plen).reshape(-1), bitorder)


def tree_masks_packed(ancs, plens, bitorder: str = "little"):
    """A batch of requests as segments: (bytes, byte indptr)."""
    parts, new = [], [0]
    for anc, plen in zip(ancs, plens):
        p = tree_mask_packed(anc, int(plen), bitorder)
        parts.append(p)
        new.append(new[-1] + p.size)
    packed = np.concatenate(parts) if parts else np.zeros(0, dtype=np.uint8)
    return packed, np.asarray(new, dtype=np.int64)
