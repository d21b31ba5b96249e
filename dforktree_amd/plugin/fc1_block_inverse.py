"""Drop-in for dforktree/fc1_block_inverse.py on MI355X.

``invert16`` / ``invert32`` / ``invert64`` keep the reference's launch form
``invert32[grid](X, N, num_warps=4, num_stages=1)`` (fc1_block_inverse.py:36-83,
called at tree_kernels.py:206): matrix ``pid`` of ``grid[0]`` lives at
``X + pid*N*N`` and holds A (its strict lower triangle is used); it is
replaced in place by (I + A)^-1 with a zero upper triangle.

The gfx950 kernel is one wave64 per matrix doing an exact forward
substitution with each lane owning one column; the reference's 16x16 block
split with tf32x3 merges is a Triton tiling choice, not part of the result.
"""
from __future__ import annotations

import torch

try:
    from dforktree_amd import ops as _ops
    from dforktree_amd import _lib
except ImportError:  # bare import, with the package itself not on sys.path
    import pathlib
    import sys
    sys.path.append(str(pathlib.Path(__file__).resolve().parents[2]))
    from dforktree_amd import ops as _ops
    from dforktree_amd import _lib


class _Invert:
    def __init__(self, n: int):
        self.n = n

    def __getitem__(self, grid):
        mats = int(grid[0] if isinstance(grid, (tuple, list)) else grid)

        def launch(P, N, num_warps=4, num_stages=1):
            if int(N) != self.n:
                raise ValueError(f"invert{self.n} called with N={N}")
            if P.dtype != torch.float32 or not P.is_contiguous() or P.numel() < mats * self.n * self.n:
                raise ValueError("P must be a contiguous float32 buffer holding grid[0] NxN matrices")
            _lib.check("dft_block_inverse",
                       _lib.load().dft_block_inverse(P.data_ptr(), mats, self.n, self.n * self.n,
                                                     _ops._stream(P.device)))
        return launch


invert16 = _Invert(16)
invert32 = _Invert(32)
invert64 = _Invert(64)
