"""MI355X-native (gfx950) GDN tree-verify path of DForkTree.

Public pieces:

* ``dforktree_amd.ops``        batched / packed operators over the HIP C ABI
  (tree_verify, tree_conv, tree_commit, tree_struct, block_inverse_);
* ``dforktree_amd.plugin``     the reference-named drop-in modules
  (``tree_kernels``, ``fc1_block_inverse``, ``fc1_fused``, ``fc1_conv``,
  ``fc1_plan``), alone in one directory for the plugin's bare imports;
* ``dforktree_amd.builder``    ``tree_struct`` / ``tree_links`` for the draft
  builder (exact ancestor closure);
* ``dforktree_amd.synth``      seeded synthetic workloads;
* ``dforktree_amd.build``      the hipcc build of libdforktree_amd.so.
"""
__version__ = "0.1.0"
