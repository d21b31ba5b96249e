"""ctypes binding of libdforktree_amd.so (the C ABI in include/dforktree_amd.h).

The structures below mirror the header field for field.  The library is
loaded from this directory only; when it is missing every entry point raises
``LibraryMissing`` -- there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdforktree_amd.so"

DFT_OK, DFT_ERR_INVALID, DFT_ERR_UNSUPPORTED, DFT_ERR_LAUNCH = 0, 1, 2, 3
DFT_F32, DFT_BF16, DFT_F16, DFT_I32, DFT_I64 = 0, 1, 2, 3, 4
DFT_VERIFY_AUX_K_PER_KHEAD = 1
DFT_COMMIT_KV, DFT_COMMIT_CHECK_ANC, DFT_COMMIT_LEN_IS_LAST = 1, 2, 4
DFT_STATUS_SPAN, DFT_STATUS_PATH, DFT_STATUS_WALK = 1, 2, 4
ABI_VERSION = 5

i32, i64, f32, vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p


class VerifyArgs(C.Structure):
    _fields_ = [
        ("batch", i32), ("n_nodes", i32), ("hk", i32), ("hv", i32), ("dk", i32), ("dv", i32),
        ("scale", f32), ("flags", i32),
        ("y", vp), ("y_row_stride", i64), ("cu_seqlens", vp),
        ("a", vp), ("a_row_stride", i64), ("a_dtype", i32),
        ("b", vp), ("b_row_stride", i64), ("b_dtype", i32),
        ("A_log", vp), ("A_log_dtype", i32),
        ("dt_bias", vp), ("dt_bias_dtype", i32),
        ("neg_exp_A", vp),
        ("anc_f32", vp), ("anc_row_stride", i64), ("anc_req_stride", i64),
        ("anc_bits", vp),
        ("state", vp), ("state_slot_stride", i64), ("state_h_stride", i64),
        ("state_k_stride", i64), ("state_v_stride", i64),
        ("state_indices", vp), ("state_indices_dtype", i32),
        ("o", vp), ("o_row_stride", i64), ("o_h_stride", i64), ("o_dtype", i32),
        ("aux_k", vp), ("aux_k_h_stride", i64), ("aux_k_row_stride", i64),
        ("aux_v", vp), ("aux_v_h_stride", i64), ("aux_v_row_stride", i64),
        ("aux_g", vp), ("aux_g_h_stride", i64), ("aux_g_row_stride", i64),
        ("status", vp),
        ("size_order", vp),
    ]


class PendingArgs(C.Structure):
    _fields_ = [
        ("path_cols", i32), ("k_head_div", i32), ("prev_n_nodes", i32),
        ("path", vp), ("path_req_stride", i64), ("path_dtype", i32),
        ("path_len", vp), ("path_len_dtype", i32),
        ("prev_cu_seqlens", vp),
        ("keys", vp), ("k_h_stride", i64), ("k_row_stride", i64),
        ("values", vp), ("v_h_stride", i64), ("v_row_stride", i64),
        ("gains", vp), ("g_h_stride", i64), ("g_row_stride", i64),
        ("key_rows", vp), ("kr_h_stride", i64), ("kr_row_stride", i64),
        ("value_rows", vp), ("vr_h_stride", i64), ("vr_row_stride", i64),
        ("prev_b", vp), ("pb_row_stride", i64), ("prev_b_dtype", i32),
        ("prev_anc_bits", vp),
    ]


class ConvArgs(C.Structure):
    _fields_ = [
        ("batch", i32), ("n_nodes", i32), ("channels", i32), ("width", i32), ("silu", i32),
        ("x", vp), ("x_req_stride", i64), ("x_node_stride", i64), ("x_chan_stride", i64), ("x_dtype", i32),
        ("conv_state", vp), ("cs_slot_stride", i64), ("cs_chan_stride", i64), ("cs_col_stride", i64),
        ("cs_dtype", i32),
        ("cs_indices", vp), ("cs_indices_dtype", i32),
        ("weight", vp), ("w_chan_stride", i64), ("w_tap_stride", i64), ("w_dtype", i32),
        ("bias", vp), ("bias_dtype", i32),
        ("cidx", vp), ("cidx_req_stride", i64), ("cidx_node_stride", i64), ("cidx_dtype", i32),
        ("y", vp), ("y_req_stride", i64), ("y_node_stride", i64), ("y_dtype", i32),
        ("iw", vp), ("iw_slot_stride", i64), ("iw_node_stride", i64), ("iw_chan_stride", i64),
        ("iw_col_stride", i64), ("iw_dtype", i32),
        ("iw_indices", vp), ("iw_indices_dtype", i32),
    ]


class CommitArgs(C.Structure):
    _fields_ = [
        ("n_layers", i32), ("batch", i32), ("hv", i32), ("dk", i32), ("dv", i32),
        ("n_nodes", i32), ("path_cols", i32), ("n_ends", i32), ("flags", i32), ("k_head_div", i32),
        ("path", vp), ("path_req_stride", i64), ("path_dtype", i32),
        ("path_len", vp), ("path_len_dtype", i32),
        ("ends", vp), ("ends_req_stride", i64), ("ends_dtype", i32),
        ("anc_bits", vp), ("anc_f32", vp), ("anc_row_stride", i64), ("anc_req_stride", i64),
        ("cu_seqlens", vp),
        ("keys", vp), ("k_layer_stride", i64), ("k_h_stride", i64), ("k_row_stride", i64),
        ("values", vp), ("v_layer_stride", i64), ("v_h_stride", i64), ("v_row_stride", i64),
        ("gains", vp), ("g_layer_stride", i64), ("g_h_stride", i64), ("g_row_stride", i64),
        ("src", vp), ("src_layer_stride", i64), ("src_slot_stride", i64), ("src_h_stride", i64),
        ("src_row_stride", i64), ("src_col_stride", i64),
        ("src_slots", vp), ("src_slots_dtype", i32),
        ("dst", vp), ("dst_layer_stride", i64), ("dst_slot_stride", i64), ("dst_node_stride", i64),
        ("dst_h_stride", i64), ("dst_row_stride", i64), ("dst_col_stride", i64),
        ("dst_slots", vp), ("dst_slots_dtype", i32),
        ("status", vp),
    ]


class TreeArgs(C.Structure):
    _fields_ = [
        ("batch", i32), ("n_nodes", i32), ("kc", i32),
        ("parent", vp), ("parent_dtype", i32),
        ("cu_seqlens", vp),
        ("anc_bits", vp),
        ("anc_f32", vp), ("anc_row_stride", i64), ("anc_req_stride", i64),
        ("depth", vp), ("depth_dtype", i32),
        ("cidx", vp), ("cidx_dtype", i32),
        ("nxt", vp), ("sib", vp), ("link_dtype", i32),
        ("status", vp),
    ]


class AncPackArgs(C.Structure):
    _fields_ = [
        ("batch", i32), ("n_nodes", i32),
        ("anc", vp), ("anc_row_stride", i64), ("anc_req_stride", i64),
        ("anc_bits", vp),
    ]


class PackbitsArgs(C.Structure):
    _fields_ = [
        ("n_segments", i32), ("bit_order", i32),
        ("x", vp), ("n", i64),
        ("indptr", vp), ("indptr_dtype", i32),
        ("out", vp), ("out_capacity", i64),
        ("out_indptr", vp), ("out_indptr_dtype", i32),
        ("status", vp),
    ]


class MaskArgs(C.Structure):
    _fields_ = [
        ("batch", i32), ("n_nodes", i32), ("bit_order", i32),
        ("cu_seqlens", vp),
        ("anc_bits", vp),
        ("prefix_len", vp), ("prefix_len_dtype", i32),
        ("out", vp), ("out_capacity", i64),
        ("out_indptr", vp), ("out_indptr_dtype", i32),
        ("status", vp),
    ]


DFT_BITS_LITTLE, DFT_BITS_BIG = 0, 1

EXPORTS = ("dft_tree_verify", "dft_tree_commit_verify", "dft_tree_conv", "dft_tree_commit", "dft_tree_struct",
           "dft_anc_pack", "dft_block_inverse", "dft_packbits", "dft_tree_mask_pack", "dft_size_order",
           "dft_error_string", "dft_abi_version")


class LibraryMissing(RuntimeError):
    pass


class DftError(RuntimeError):
    def __init__(self, fn, status, msg):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


_lib = None


def load() -> C.CDLL:
    """Load the in-tree library (once) and declare the entry points."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -m dforktree_amd.build` (hipcc, gfx950)")
    lib = C.CDLL(str(LIB_PATH))
    for name, argt in (("dft_tree_verify", [C.POINTER(VerifyArgs), vp]),
                       ("dft_tree_commit_verify", [C.POINTER(VerifyArgs), C.POINTER(PendingArgs), vp]),
                       ("dft_tree_conv", [C.POINTER(ConvArgs), vp]),
                       ("dft_tree_commit", [C.POINTER(CommitArgs), vp]),
                       ("dft_tree_struct", [C.POINTER(TreeArgs), vp]),
                       ("dft_anc_pack", [C.POINTER(AncPackArgs), vp]),
                       ("dft_packbits", [C.POINTER(PackbitsArgs), vp]),
                       ("dft_tree_mask_pack", [C.POINTER(MaskArgs), vp]),
                       ("dft_block_inverse", [vp, i32, i32, i64, vp]),
                       ("dft_size_order", [vp, i32, i32, vp, vp])):
        fn = getattr(lib, name)
        fn.argtypes = argt
        fn.restype = C.c_int
    lib.dft_error_string.argtypes = [C.c_int]
    lib.dft_error_string.restype = C.c_char_p
    lib.dft_abi_version.argtypes = []
    lib.dft_abi_version.restype = C.c_int
    if lib.dft_abi_version() != ABI_VERSION:
        raise LibraryMissing(f"{LIB_PATH} has ABI version {lib.dft_abi_version()}, this binding needs {ABI_VERSION}; "
                             "rebuild it (python -m dforktree_amd.build)")
    _lib = lib
    return lib


def check(fn_name: str, status: int) -> None:
    if status != DFT_OK:
        msg = load().dft_error_string(status).decode()
        raise DftError(fn_name, status, msg)
