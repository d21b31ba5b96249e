"""The reference-named drop-in modules, alone in one directory.

DForkTree's plugin imports its path modules by bare name after putting its
own directory on ``sys.path`` (fc1_plugin.py:27; fc1_fused.py:10,
fc1_conv.py:5, tree_kernels.py:205, fc1_branch64.py:27, :37).  Putting
``PATH`` (this directory) in front of it makes exactly these five names
resolve here:

* ``tree_kernels``       tree_kernels.py (verify, conv, in-place commit)
* ``fc1_block_inverse``  fc1_block_inverse.py (invert16/32/64)
* ``fc1_fused``          fc1_fused.py (Context, CTX, snapshots, install)
* ``fc1_conv``           fc1_conv.py (conv, install)
* ``fc1_plan``           fc1_plan.py (HOST_KV_LEN, install)

Every other name the reference imports -- ``tree_ops``, ``ngram_gpu``,
``fc1_builder``, ``fc1_branch64``, ``fc1_verify``, ``fc1_dflash_worker``,
``fc1_plugin`` -- keeps resolving to the reference's own file, because
nothing else lives here.  Import these modules by one name only (the bare
one, as the plugin does): ``fc1_fused`` and ``dforktree_amd.plugin.fc1_fused``
would be two modules with two ``CTX`` singletons.
"""
import os

PATH = os.path.dirname(os.path.abspath(__file__))

# the module names above, and only those, are files of this directory
MODULES = ("tree_kernels", "fc1_block_inverse", "fc1_fused", "fc1_conv", "fc1_plan")
