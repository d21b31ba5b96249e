"""The draft-tree builder's tree-structure step on MI355X.

``tree_struct(parent_full, Kc)`` returns (Anc [N,N] fp32, depth [N] int64,
cidx [N,Kc] int64) as tree_ops.py:68-89 does, computed by one gfx950 wave
per tree.  The ancestor closure is exact at every depth: the reference's
five squarings (tree_ops.py:75-79) stop at 31 edges, so the two agree bit
for bit up to 31 edges and only this one is right for 64-node chains.
``tree_links(parent)`` gives the builder's first-child / next-sibling links
(fc1_builder.py:41-47).

This module is deliberately not named ``tree_ops``: the reference's
``tree_ops`` also holds the draft search (``beam_tree``, ``ngram_path_fn``,
tree_ops.py:7-66) that ``fc1_builder`` calls, and that stays the
reference's.  A builder opts in to the exact closure by calling this
``tree_struct`` in place of ``TO.tree_struct`` (fc1_builder.py:39).  Both
functions launch on the current stream and read nothing back to the host,
so they can run inside the builder's graph capture (fc1_builder.py:20-22).
"""
from __future__ import annotations

from . import ops as _ops


def tree_struct(parent_full, Kc):
    """Node 0 is the root; for i >= 1 the parent is max(parent_full[i], 0)."""
    r = _ops.tree_struct(parent_full.reshape(-1), Kc, want=("anc", "depth", "cidx"))
    return r["anc"][0], r["depth"], r["cidx"]


def tree_links(parent):
    """(nxt, sib): first child and next sibling of every node, -1 for none."""
    r = _ops.tree_struct(parent.reshape(-1), 1, want=("nxt", "sib"))
    return r["nxt"], r["sib"]
