"""CPU oracle for the GDN tree-verify path.

TEST INFRASTRUCTURE ONLY. This package is what the tests compare against,
never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (``dforktree_amd``) runs the HIP
kernels and raises when the HIP library is missing; it never calls in here.

Contents (``oracle.gdn_tree``):

* ``tree_struct``            exact ancestor closure / depth / conv gather columns
                             (tree_ops.py:68-89), ``tree_links`` (fc1_builder.py:41-47)
* ``prepare`` / ``block_invert`` / ``finish`` / ``tree_gdn_split``
                             fp32 restatement of the split verify
                             (tree_kernels.py:135-208, fc1_block_inverse.py:10-83)
* ``tree_gdn_neumann``       the single-kernel variant with its Neumann-16
                             inverse (tree_kernels.py:35-81)
* ``recurrent_f64``          independent fp64 per-node recurrence (the pin)
* ``tree_conv``              tree-parent causal conv1d (fc1_conv.py:7-27,
                             tree_kernels.py:17-33)
* ``closed_commit`` / ``snapshot_commit`` closed-form accepted-path commit
                             (tree_kernels.py:111-127, fc1_fused.py:26-49)

``oracle.gdn_tree_torch``: the split verify and the closed commit as batched
PyTorch fp32 CPU ops (the CPU baseline bench.py times), pinned against
``oracle.gdn_tree``.

``oracle.mask``: ``packbits`` / ``segment_packbits`` (numpy.packbits per
segment, as flashinfer packs the custom mask for fc1_plan.py:26) and
``tree_mask`` / ``tree_mask_packed`` (the mask of fc1_branch64.py:39).

Pinning status of every function is listed in the module docstrings of
``oracle.gdn_tree`` and ``oracle.mask``.
"""
