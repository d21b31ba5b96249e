"""The C ABI boundary, checked on the CPU: the library loads, exports every
entry point the header declares, the ctypes descriptors match the C structs
byte for byte (offsets computed by gcc from the header), and argument
validation rejects bad descriptors before any launch."""
import ctypes
import json
import re
import subprocess

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "dforktree_amd.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^DFT_API\s+(?:int|const char\*)\s+(dft_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    from dforktree_amd import _lib
    names = declared_functions()
    assert set(names) == set(_lib.EXPORTS)
    lib = _lib.load()
    for n in names:
        assert getattr(lib, n) is not None
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == set(names), "only the C ABI is exported"
    assert lib.dft_abi_version() == _lib.ABI_VERSION == 5


@pytest.fixture(scope="module")
def c_layouts(tmp_path_factory):
    from dforktree_amd import _lib
    structs = {"dft_verify_args": _lib.VerifyArgs, "dft_pending_commit": _lib.PendingArgs, "dft_conv_args": _lib.ConvArgs,
               "dft_commit_args": _lib.CommitArgs, "dft_tree_args": _lib.TreeArgs,
               "dft_packbits_args": _lib.PackbitsArgs, "dft_mask_args": _lib.MaskArgs,
               "dft_anc_pack_args": _lib.AncPackArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {",
             'printf("{");']
    first = True
    for cname, py in structs.items():
        for f, _ in py._fields_:
            sep = "" if first else ","
            first = False
            lines.append(f'printf("{sep}\\"{cname}.{f}\\": %zu", offsetof({cname}, {f}));')
        lines.append(f'printf(",\\"{cname}.__size__\\": %zu", sizeof({cname}));')
    lines += ['printf("}");', "return 0; }"]
    d = tmp_path_factory.mktemp("abi")
    src, exe = d / "layout.c", d / "layout"
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    return json.loads(subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout), structs


def test_ctypes_structs_match_c_layout(c_layouts):
    from dforktree_amd import _lib
    layout, structs = c_layouts
    # the status words, then the size-order records, were appended: every earlier field kept its offset
    assert [f for f, _ in _lib.VerifyArgs._fields_[-2:]] == ["status", "size_order"]
    assert _lib.CommitArgs._fields_[-1][0] == "status"
    # ABI 5 appended the previous step's ancestry rows (the walk check) to the pending commit
    assert _lib.PendingArgs._fields_[-1][0] == "prev_anc_bits"
    assert _lib.PendingArgs._fields_[-4][0] == "prev_b"
    for cname, py in structs.items():
        assert ctypes.sizeof(py) == layout[f"{cname}.__size__"], cname
        for f, _ in py._fields_:
            assert getattr(py, f).offset == layout[f"{cname}.{f}"], f"{cname}.{f}"


def test_validation_rejects_bad_descriptors_without_launching():
    """Every check below fails on the host before any HIP call."""
    from dforktree_amd import _lib
    lib = _lib.load()
    v = _lib.VerifyArgs()
    v.batch, v.n_nodes, v.hk, v.hv, v.dk, v.dv = 1, 32, 2, 4, 64, 128
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_UNSUPPORTED  # dk != 128
    v.dk = 128
    v.hv = 3
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_INVALID      # hv % hk
    v.hv, v.n_nodes = 4, 65
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_UNSUPPORTED  # > 64 nodes
    v.n_nodes = 32
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_INVALID      # null pointers
    v.batch = 0
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_OK                # empty batch: no-op
    v.batch, v.n_nodes = 1, 32
    assert lib.dft_size_order(None, 1, 64, 16, None) == _lib.DFT_ERR_INVALID        # no cu_seqlens
    assert lib.dft_size_order(16, 1, 65, 16, None) == _lib.DFT_ERR_INVALID          # > 64 nodes
    assert lib.dft_size_order(16, -1, 64, 16, None) == _lib.DFT_ERR_INVALID         # batch
    assert lib.dft_size_order(16, 1, 64, 8, None) == _lib.DFT_ERR_INVALID           # records: 16 B
    pc = _lib.PendingArgs()
    pc.path_cols, pc.k_head_div, pc.prev_n_nodes, pc.path_dtype = 16, 1, 32, _lib.DFT_I32
    assert lib.dft_tree_commit_verify(ctypes.byref(v), None, None) == _lib.DFT_ERR_INVALID  # null pointers
    v.y = v.a = v.b = v.A_log = v.dt_bias = v.state = v.o = v.anc_bits = 16
    v.y_row_stride, v.state_k_stride, v.state_v_stride = 8, 1, 128
    v.size_order = 16
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_INVALID       # size order, not packed
    v.cu_seqlens, v.size_order = 16, 8
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_INVALID       # records: 16 B
    v.cu_seqlens, v.size_order = None, None
    assert lib.dft_tree_commit_verify(ctypes.byref(v), None, None) == _lib.DFT_ERR_INVALID  # no pending
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID
    pc.path = pc.keys = pc.values = pc.gains = 16
    pc.key_rows = 16
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # keys twice
    pc.keys, pc.key_rows = None, 12
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # raw rows: 8 B
    pc.key_rows, pc.kr_row_stride = 16, 6
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # stride % 4
    pc.keys, pc.key_rows, pc.kr_row_stride = 16, None, 0
    pc.value_rows = 16
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # values twice
    pc.values = None
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # no b gates
    pc.prev_b, pc.prev_b_dtype = 16, 99
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # b dtype
    pc.values, pc.value_rows, pc.prev_b, pc.prev_b_dtype = 16, None, None, 0
    pc.path_cols = 17
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_UNSUPPORTED
    pc.path_cols = 0  # the kernel pads from entry path_cols - 1: at least one column
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID
    pc.path_cols, v.state_k_stride, v.state_v_stride = 16, 128, 1  # k-major state: no 16-byte rows
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_UNSUPPORTED
    v.batch = 0
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_OK  # empty: no-op
    # n_nodes 0 with requests: the fused entry still commits (it needs the state and the pending path, not the
    # rows), the plain verify has nothing to do
    v.batch, v.n_nodes, v.state_k_stride, v.state_v_stride = 1, 0, 1, 128
    v.y = v.a = v.b = v.o = v.anc_bits = None
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_OK
    v.state = None
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # no state
    v.state = 16
    pc.path = None
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_INVALID  # no path
    pc.path, v.state_k_stride, v.state_v_stride = 16, 128, 1
    assert lib.dft_tree_commit_verify(ctypes.byref(v), ctypes.byref(pc), None) == _lib.DFT_ERR_UNSUPPORTED
    c = _lib.CommitArgs()
    c.n_layers, c.batch, c.hv, c.dk, c.dv, c.n_nodes, c.path_cols, c.n_ends, c.k_head_div = 1, 1, 4, 128, 128, 32, 16, 3, 1
    assert lib.dft_tree_commit(ctypes.byref(c), None) == _lib.DFT_ERR_INVALID       # n_ends
    c.n_ends = 2
    c.path = c.keys = c.values = c.gains = c.src = c.dst = 16
    assert lib.dft_tree_commit(ctypes.byref(c), None) == _lib.DFT_ERR_INVALID       # 2 ends in place
    c.n_ends, c.path_cols = 1, 0
    assert lib.dft_tree_commit(ctypes.byref(c), None) == _lib.DFT_ERR_INVALID       # no path column
    c.path_cols = 16
    t = _lib.TreeArgs()
    t.batch, t.n_nodes, t.kc = 1, 65, 4
    assert lib.dft_tree_struct(ctypes.byref(t), None) == _lib.DFT_ERR_INVALID
    ap = _lib.AncPackArgs()
    ap.batch, ap.n_nodes = 1, 65
    assert lib.dft_anc_pack(ctypes.byref(ap), None) == _lib.DFT_ERR_INVALID         # > 64 nodes
    ap.n_nodes = 32
    assert lib.dft_anc_pack(ctypes.byref(ap), None) == _lib.DFT_ERR_INVALID         # null pointers
    ap.batch = 0
    assert lib.dft_anc_pack(ctypes.byref(ap), None) == _lib.DFT_OK                  # empty: no-op
    k = _lib.ConvArgs()
    k.batch, k.n_nodes, k.channels, k.width = 1, 4, 8, 9
    assert lib.dft_tree_conv(ctypes.byref(k), None) == _lib.DFT_ERR_UNSUPPORTED
    assert lib.dft_block_inverse(None, 1, 65, 65 * 65, None) == _lib.DFT_ERR_INVALID
    pb = _lib.PackbitsArgs()
    pb.n, pb.bit_order = 8, 2
    assert lib.dft_packbits(ctypes.byref(pb), None) == _lib.DFT_ERR_INVALID        # bit order
    pb.bit_order = _lib.DFT_BITS_LITTLE
    assert lib.dft_packbits(ctypes.byref(pb), None) == _lib.DFT_ERR_INVALID        # null pointers
    pb.x = pb.out = 16
    pb.out_capacity = -1
    assert lib.dft_packbits(ctypes.byref(pb), None) == _lib.DFT_ERR_INVALID        # capacity
    pb.out_capacity, pb.indptr, pb.indptr_dtype, pb.n_segments = 8, 16, _lib.DFT_I32, 70000
    assert lib.dft_packbits(ctypes.byref(pb), None) == _lib.DFT_ERR_UNSUPPORTED    # > 65535 segments
    pb.n_segments = 0
    assert lib.dft_packbits(ctypes.byref(pb), None) == _lib.DFT_OK                 # no segment: no-op
    mk = _lib.MaskArgs()
    mk.batch, mk.n_nodes = 1, 65
    assert lib.dft_tree_mask_pack(ctypes.byref(mk), None) == _lib.DFT_ERR_INVALID  # > 64 nodes
    mk.n_nodes = 32
    assert lib.dft_tree_mask_pack(ctypes.byref(mk), None) == _lib.DFT_ERR_INVALID  # null pointers
    mk.anc_bits = mk.prefix_len = mk.out = 16
    mk.prefix_len_dtype = 7
    assert lib.dft_tree_mask_pack(ctypes.byref(mk), None) == _lib.DFT_ERR_INVALID  # prefix dtype
    mk.batch = 0
    assert lib.dft_tree_mask_pack(ctypes.byref(mk), None) == _lib.DFT_OK           # empty batch: no-op
    assert lib.dft_error_string(2) == b"unsupported configuration"


def test_validation_refuses_grids_past_the_launch_limit():
    """A grid's x extent counts work-items in 32 bits, so at most
    (2**32 - 1) // 256 workgroups of 256 threads: larger batches are refused
    as unsupported on the host instead of failing at launch."""
    from dforktree_amd import _lib
    lib = _lib.load()
    limit = (2**32 - 1) // 256
    v = _lib.VerifyArgs()
    v.n_nodes, v.hk, v.hv, v.dk, v.dv = 32, 1, 8, 128, 128
    v.y = v.a = v.b = v.A_log = v.dt_bias = v.state = v.o = v.anc_bits = 16
    v.a_dtype = v.b_dtype = v.dt_bias_dtype = v.A_log_dtype = v.o_dtype = _lib.DFT_F32
    v.y_row_stride = 8
    v.batch = limit // 8 + 1  # batch * hv workgroups
    assert lib.dft_tree_verify(ctypes.byref(v), None) == _lib.DFT_ERR_UNSUPPORTED
    c = _lib.CommitArgs()
    c.n_layers, c.batch, c.hv, c.dk, c.dv, c.n_nodes, c.path_cols, c.n_ends, c.k_head_div = 24, 1, 32, 128, 128, 32, 16, 1, 1
    c.path = c.keys = c.values = c.gains = c.src = c.dst = 16
    c.path_dtype = _lib.DFT_I32
    c.batch = limit // (24 * 32) + 1  # layers * batch * heads workgroups
    assert lib.dft_tree_commit(ctypes.byref(c), None) == _lib.DFT_ERR_UNSUPPORTED
    k = _lib.ConvArgs()
    k.batch, k.n_nodes, k.channels, k.width = 65535, 65535, 8192, 4  # 16 workgroups per (request, node)
    k.x = k.conv_state = k.weight = k.cidx = k.y = 16
    k.cidx_dtype = _lib.DFT_I32
    assert lib.dft_tree_conv(ctypes.byref(k), None) == _lib.DFT_ERR_UNSUPPORTED
    assert lib.dft_block_inverse(16, 2**31 - 1, 64, 64 * 64, None) == _lib.DFT_ERR_UNSUPPORTED  # 64-thread groups
    t = _lib.TreeArgs()
    t.batch, t.n_nodes, t.kc = 2**31 - 1, 32, 4  # four requests per workgroup
    t.parent, t.parent_dtype = 16, _lib.DFT_I32
    assert lib.dft_tree_struct(ctypes.byref(t), None) == _lib.DFT_ERR_UNSUPPORTED


def test_python_layer_refuses_cpu_tensors():
    """No CPU fallback: the operators take device tensors only."""
    import torch
    from dforktree_amd import ops
    x = torch.zeros(4, 4)
    with pytest.raises(ValueError, match="GPU tensors"):
        ops.block_inverse_(x)


def test_stream_copy_library_is_outside_the_c_abi():
    """The bench's copy calibration kernel lives in its own library, exports
    one symbol and rejects bad arguments before any launch."""
    from dforktree_amd import build
    assert build.CALIB_LIB.exists()
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.CALIB_LIB)], capture_output=True, text=True).stdout
    assert {l.split()[-1] for l in out.splitlines() if " T " in l} == {"dft_calib_stream_copy"}
    lib = ctypes.CDLL(str(build.CALIB_LIB))
    f = lib.dft_calib_stream_copy
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
    assert f(None, ctypes.c_void_p(16), 16, None) == 1
    assert f(ctypes.c_void_p(16), ctypes.c_void_p(32), 24, None) == 1   # not a multiple of 16
    assert f(ctypes.c_void_p(16), ctypes.c_void_p(40), 16, None) == 1   # misaligned destination
    assert f(ctypes.c_void_p(16), ctypes.c_void_p(32), 0, None) == 1
