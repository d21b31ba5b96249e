"""The plugin binding (one line added to fc1_plugin.register), resolved the way
the plugin resolves it: fc1_plugin.register puts the reference's own directory first on
sys.path (fc1_plugin.py:27), then the one added line puts
``dforktree_amd.plugin.PATH`` in front of it.  Every bare module name the
reference's files import must then resolve -- the five replaced ones here,
every other one to the reference's own file -- with the attributes those
files use.

The reference directory is played by stand-in files with the reference's
module names (no reference code is imported or read).  The check runs in a
fresh interpreter so that sys.path and sys.modules start clean.
"""
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

# the modules of the reference's dforktree/ directory
REFERENCE_MODULES = ("fc1_block_inverse", "fc1_branch64", "fc1_builder", "fc1_conv", "fc1_dflash_worker", "fc1_fused",
                     "fc1_plan", "fc1_plugin", "fc1_verify", "ngram_gpu", "tree_kernels", "tree_ops")
REPLACED = ("tree_kernels", "fc1_block_inverse", "fc1_fused", "fc1_conv", "fc1_plan")

# Stand-ins: each carries a marker and the names the other reference files use,
# and makes the same bare imports its reference file makes.
STANDINS = {
    "tree_ops": "def beam_tree(*a, **k): pass\ndef ngram_path_fn(*a, **k): pass\ndef tree_struct(*a, **k): pass\n",
    "ngram_gpu": "class NGramGPU: pass\n",
    # fc1_builder.py:5-6
    "fc1_builder": "import tree_ops as TO\nfrom ngram_gpu import NGramGPU\nclass Builder: pass\n",
    # fc1_branch64.py:18, :27, :37
    "fc1_branch64": ("def verify_branch():\n    from fc1_builder import Builder\n    import fc1_fused\n"
                     "    import fc1_plan\n    return Builder, fc1_fused, fc1_plan\n"),
    "fc1_verify": "class ChainTreeVerifyInput: pass\n",
    # fc1_dflash_worker.py:32
    "fc1_dflash_worker": "from fc1_verify import ChainTreeVerifyInput as DFlashVerifyInput\n",
    "fc1_plugin": "def register(): pass\n",
    "tree_kernels": "",
    "fc1_block_inverse": "",
    "fc1_fused": "",
    "fc1_conv": "",
    "fc1_plan": "",
}

CHECK = r'''
import importlib, os, sys
standin, root, installed = sys.argv[1], sys.argv[2], sys.argv[3] == "1"
sys.path.insert(0, standin)                      # fc1_plugin.py:27
if installed:
    sys.path.append(root)                        # the package importable, as when installed
    import dforktree_amd.plugin                  # the line added to fc1_plugin.register
    sys.path.insert(0, dforktree_amd.plugin.PATH)
    plugin_dir = dforktree_amd.plugin.PATH
else:                                            # the directory alone on sys.path
    plugin_dir = os.path.join(root, "dforktree_amd", "plugin")
    sys.path.insert(0, plugin_dir)

REPLACED = %(replaced)r
OTHERS = %(others)r
for name in REPLACED:
    mod = importlib.import_module(name)
    assert os.path.dirname(os.path.abspath(mod.__file__)) == plugin_dir, (name, mod.__file__)
    assert not hasattr(mod, "ORIGIN"), name
for name in OTHERS:
    mod = importlib.import_module(name)
    assert getattr(mod, "ORIGIN", None) == "reference-standin", (name, mod.__file__)
    assert os.path.dirname(os.path.abspath(mod.__file__)) == standin, (name, mod.__file__)

# fc1_builder.py:5-6, :31, :37, :39 -- the draft search stays the reference's
import fc1_builder
TO = fc1_builder.TO
assert TO is sys.modules["tree_ops"] and TO.ORIGIN == "reference-standin"
for attr in ("ngram_path_fn", "beam_tree", "tree_struct"):
    assert callable(getattr(TO, attr)), attr
assert fc1_builder.NGramGPU is sys.modules["ngram_gpu"].NGramGPU

# fc1_fused.py:10 and tree_kernels.py:205
import fc1_fused, fc1_conv, fc1_plan, tree_kernels, fc1_block_inverse
assert fc1_fused.TK is tree_kernels
for attr in ("tree_gdn_split", "tree_gdn_fused", "tree_conv_fused", "closed_commit", "available", "_pow2"):
    assert callable(getattr(tree_kernels, attr)), attr
from fc1_block_inverse import invert64, invert32, invert16
assert invert64.n == 64 and invert32.n == 32 and invert16.n == 16

# fc1_conv.py:5, :34-44: one fc1_fused module object, with the fields the conv uses
assert fc1_conv.F is fc1_fused
for attr in ("NATIVE_REFERENCE", "NN", "BS", "CTX", "Context", "snapshots", "install", "LAYER_STATS",
             "COLLECT_LAYER"):
    assert hasattr(fc1_fused, attr), attr
ctx = fc1_fused.Context(device="cpu")
for attr in ("anc", "keys", "values", "gains", "layers", "inter_indices", "current_mixed"):
    assert hasattr(ctx, attr), attr
assert tuple(ctx.anc.shape) == (fc1_fused.NN, fc1_fused.NN)

# fc1_branch64.py:18-30, :37-38
import fc1_branch64
Builder, F, P = fc1_branch64.verify_branch()
assert Builder is fc1_builder.Builder and F is fc1_fused and P is fc1_plan
F.CTX = ctx
F.CTX.anc.copy_(ctx.anc)
F.CTX.cidx = fc1_conv.default_cidx(F.NN, "cpu")
P.HOST_KV_LEN = 7

# fc1_plugin.py:29-34 and fc1_dflash_worker.py:32
from fc1_fused import install as a
from fc1_conv import install as b
from fc1_plan import install as c
import fc1_dflash_worker
assert fc1_dflash_worker.DFlashVerifyInput is sys.modules["fc1_verify"].ChainTreeVerifyInput

# nothing from the reference tree was loaded
for name, mod in list(sys.modules.items()):
    f = getattr(mod, "__file__", None) or ""
    assert "/root/reference" not in f, (name, f)
print("bare imports resolved")
'''


def _standin_dir(tmp_path):
    d = tmp_path / "dforktree"
    d.mkdir()
    (d / "__init__.py").write_text("")
    for name, body in STANDINS.items():
        (d / f"{name}.py").write_text("ORIGIN = 'reference-standin'\n" + body)
    return d


def test_standins_cover_every_reference_module():
    assert set(STANDINS) == set(REFERENCE_MODULES)


def test_plugin_directory_holds_only_the_replaced_modules():
    from dforktree_amd import plugin
    files = sorted(p.stem for p in Path(plugin.PATH).glob("*.py") if p.stem != "__init__")
    assert files == sorted(REPLACED) == sorted(plugin.MODULES)
    assert not any(Path(plugin.PATH).glob("*.so")) and not [p for p in Path(plugin.PATH).iterdir()
                                                           if p.is_dir() and p.name != "__pycache__"]


@pytest.mark.parametrize("installed", [True, False], ids=["package-importable", "directory-only"])
def test_integration_binding_resolves_every_bare_name(tmp_path, installed):
    d = _standin_dir(tmp_path)
    others = tuple(m for m in REFERENCE_MODULES if m not in REPLACED)
    script = CHECK % dict(replaced=REPLACED, others=others)
    r = subprocess.run([sys.executable, "-c", textwrap.dedent(script), str(d), str(ROOT), "1" if installed else "0"],
                       capture_output=True, text=True, timeout=300, cwd=str(tmp_path))
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bare imports resolved" in r.stdout
