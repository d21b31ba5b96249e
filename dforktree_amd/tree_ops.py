"""Drop-in for the verify-input half of dforktree/tree_ops.py on MI355X.

``tree_struct(parent_full, Kc)`` returns (Anc [N,N] fp32, depth [N] int64,
cidx [N,Kc] int64) like tree_ops.py:68-89, computed by one gfx950 wave per
tree.  The ancestor closure is exact at every depth; the reference's five
squarings (tree_ops.py:75-79) stop at 31 edges, so the two agree bit for bit
for N <= 32 and this one is also right for the 64-node chains.

``beam_tree`` and ``ngram_path_fn`` (draft-tree search, tree_ops.py:7-66) are
not on the verify path and are not provided.
"""
from __future__ import annotations

try:
    from dforktree_amd import ops as _ops
except ImportError:  # bare import from this directory
    import pathlib
    import sys
    sys.path.insert(0, str(pathlib.Path(__file__).resolve().parents[1]))
    from dforktree_amd import ops as _ops


def tree_struct(parent_full, Kc):
    """Node 0 is the root; for i >= 1 the parent is max(parent_full[i], 0)."""
    r = _ops.tree_struct(parent_full.reshape(-1), Kc, want=("anc", "depth", "cidx"))
    return r["anc"][0], r["depth"], r["cidx"]


def tree_links(parent):
    """First-child / next-sibling links of the builder (fc1_builder.py:41-47)."""
    r = _ops.tree_struct(parent.reshape(-1), 1, want=("nxt", "sib"))
    return r["nxt"], r["sib"]
