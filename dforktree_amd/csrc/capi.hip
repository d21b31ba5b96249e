// extern "C" entry points: validate the descriptor on the host, then launch.
// No allocation, no host<->device synchronisation.
#include <stdint.h>

#include "dft_device.h"

namespace dft {
int launch_tree_verify(const dft_verify_args* a, hipStream_t stream);
int launch_tree_commit_verify(const dft_verify_args* a, const dft_pending_commit* c, hipStream_t stream);
int launch_block_inverse(float* x, int n_mats, int n, int64_t mat_stride, hipStream_t stream);
int launch_size_order(const int32_t* cu_seqlens, int batch, int n_nodes, int32_t* order, hipStream_t stream);
int launch_tree_conv(const dft_conv_args* a, hipStream_t stream);
int launch_tree_commit(const dft_commit_args* a, hipStream_t stream);
int launch_tree_struct(const dft_tree_args* a, hipStream_t stream);
int launch_anc_pack(const dft_anc_pack_args* a, hipStream_t stream);
int launch_packbits(const dft_packbits_args* a, hipStream_t stream);
int launch_tree_mask(const dft_mask_args* a, hipStream_t stream);
}  // namespace dft

namespace {

bool float_tag(int32_t t) { return t == DFT_F32 || t == DFT_BF16 || t == DFT_F16; }
bool index_tag(int32_t t) { return t == DFT_I32 || t == DFT_I64; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A grid's x extent counts work-items in 32 bits: at most this many
// workgroups of `threads` threads.
constexpr int64_t max_blocks(int threads) { return (int64_t)0xffffffffll / threads; }

// Checks shared by the verify entry points: DFT_OK to launch, DFT_ERR_* to
// refuse, or -1 when there is nothing to do.  commit_only: a launch of the
// fused entry with n_nodes 0, which commits the pending paths and verifies
// nothing, so it reads no rows, gates, ancestry or outputs.
int verify_status(const dft_verify_args* a, bool commit_only = false) {
  if (!a) return DFT_ERR_INVALID;
  if (a->batch < 0 || a->n_nodes < 0 || a->hk <= 0 || a->hv <= 0 || a->hv % a->hk != 0) return DFT_ERR_INVALID;
  if (a->dk != 128 || a->dv != 128) return DFT_ERR_UNSUPPORTED;
  if (a->n_nodes > 64) return DFT_ERR_UNSUPPORTED;
  if (a->batch == 0 || (a->n_nodes == 0 && !commit_only)) return -1;
  if (!a->state) return DFT_ERR_INVALID;
  if (a->state_indices && !index_tag(a->state_indices_dtype)) return DFT_ERR_INVALID;
  // size-order records: 16-byte records of a packed batch
  if (a->size_order && (!a->cu_seqlens || !aligned16(a->size_order))) return DFT_ERR_INVALID;
  // one workgroup per (request, v-head): 4 waves for trees of up to 32 nodes, 8 beyond
  if ((int64_t)a->batch * a->hv > max_blocks(a->n_nodes > 32 ? 512 : 256)) return DFT_ERR_UNSUPPORTED;
  if (a->n_nodes == 0) return DFT_OK;
  if (!a->y || !a->a || !a->b || !a->o) return DFT_ERR_INVALID;
  if (!a->neg_exp_A && !a->A_log) return DFT_ERR_INVALID;
  if (!a->dt_bias) return DFT_ERR_INVALID;
  if ((a->anc_f32 == nullptr) == (a->anc_bits == nullptr)) return DFT_ERR_INVALID;
  if (!float_tag(a->a_dtype) || !float_tag(a->b_dtype) || !float_tag(a->dt_bias_dtype) ||
      (a->A_log && !float_tag(a->A_log_dtype)))
    return DFT_ERR_INVALID;
  if (a->o_dtype != DFT_F32 && a->o_dtype != DFT_BF16 && a->o_dtype != DFT_F16) return DFT_ERR_INVALID;
  // q/k/v rows are copied as 16-byte pieces
  if (!aligned16(a->y) || a->y_row_stride % 8 != 0) return DFT_ERR_INVALID;
  return DFT_OK;
}

}  // namespace

extern "C" {

int dft_abi_version(void) { return DFT_ABI_VERSION; }

const char* dft_error_string(int status) {
  switch (status) {
    case DFT_OK: return "ok";
    case DFT_ERR_INVALID: return "invalid argument (pointer, size, stride, dtype or alignment)";
    case DFT_ERR_UNSUPPORTED: return "unsupported configuration";
    case DFT_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown status";
  }
}

int dft_tree_verify(const dft_verify_args* a, void* stream) {
  const int st = verify_status(a);
  if (st != DFT_OK) return st < 0 ? DFT_OK : st;
  return dft::launch_tree_verify(a, static_cast<hipStream_t>(stream));
}

int dft_tree_commit_verify(const dft_verify_args* a, const dft_pending_commit* c, void* stream) {
  // n_nodes 0 (every request's tree empty) still commits the pending paths
  const int st = verify_status(a, /*commit_only=*/true);
  if (st != DFT_OK) return st < 0 ? DFT_OK : st;
  if (!c) return DFT_ERR_INVALID;
  if (c->path_cols < 1) return DFT_ERR_INVALID;  // the kernels read entry path_cols - 1 for padding lanes
  if (c->path_cols > 16) return DFT_ERR_UNSUPPORTED;
  if (c->k_head_div <= 0 || a->hv % c->k_head_div != 0) return DFT_ERR_INVALID;
  if (!c->prev_cu_seqlens && (c->prev_n_nodes < 0 || c->prev_n_nodes > 64)) return DFT_ERR_INVALID;
  if (!c->path || !c->gains) return DFT_ERR_INVALID;
  if ((c->keys != nullptr) == (c->key_rows != nullptr)) return DFT_ERR_INVALID;  // saved keys or raw rows
  // saved values, or the raw value rows and b gates they are recomputed from
  if ((c->values != nullptr) == (c->value_rows != nullptr)) return DFT_ERR_INVALID;
  if (c->value_rows && (!c->prev_b || !float_tag(c->prev_b_dtype))) return DFT_ERR_INVALID;
  // raw key rows are read as 8-byte pieces
  if (c->key_rows && (reinterpret_cast<uintptr_t>(c->key_rows) % 8 || c->kr_row_stride % 4 || c->kr_h_stride % 4))
    return DFT_ERR_INVALID;
  if (!index_tag(c->path_dtype) || (c->path_len && !index_tag(c->path_len_dtype))) return DFT_ERR_INVALID;
  // the committed tile is written back with the same 16-byte accesses that read it
  if (a->state_k_stride != 1 || !aligned16(a->state) || a->state_v_stride % 4 || a->state_h_stride % 4 ||
      a->state_slot_stride % 4)
    return DFT_ERR_UNSUPPORTED;
  return dft::launch_tree_commit_verify(a, c, static_cast<hipStream_t>(stream));
}

int dft_size_order(const int32_t* cu_seqlens, int32_t batch, int32_t n_nodes, int32_t* order, void* stream) {
  if (batch < 0 || n_nodes < 1 || n_nodes > 64 || !cu_seqlens || !order) return DFT_ERR_INVALID;
  if (!aligned16(order)) return DFT_ERR_INVALID;  // 16-byte records
  return dft::launch_size_order(cu_seqlens, batch, n_nodes, order, static_cast<hipStream_t>(stream));
}

int dft_block_inverse(float* x, int32_t n_mats, int32_t n, int64_t mat_stride, void* stream) {
  if (n_mats < 0 || n < 0 || n > 64) return DFT_ERR_INVALID;
  if (n_mats == 0 || n == 0) return DFT_OK;
  if (!x || mat_stride < (int64_t)n * n) return DFT_ERR_INVALID;
  if (n_mats > max_blocks(64)) return DFT_ERR_UNSUPPORTED;
  return dft::launch_block_inverse(x, n_mats, n, mat_stride, static_cast<hipStream_t>(stream));
}

int dft_tree_conv(const dft_conv_args* a, void* stream) {
  if (!a) return DFT_ERR_INVALID;
  if (a->batch < 0 || a->n_nodes < 0 || a->channels < 0) return DFT_ERR_INVALID;
  if (a->width < 1 || a->width > 8) return DFT_ERR_UNSUPPORTED;
  if (a->batch == 0 || a->n_nodes == 0 || a->channels == 0) return DFT_OK;
  if (a->n_nodes > 65535 || a->batch > 65535) return DFT_ERR_UNSUPPORTED;
  // the width-4 bf16 path launches one 64-thread workgroup per (request, node, 512 channels), rounded to 8
  const int64_t pairs8 = ((int64_t)a->batch * ((a->channels + 511) / 512) + 7) / 8;
  if (pairs8 * 8 * a->n_nodes > max_blocks(64)) return DFT_ERR_UNSUPPORTED;
  if (!a->x || !a->conv_state || !a->weight || !a->cidx || !a->y) return DFT_ERR_INVALID;
  if (!float_tag(a->x_dtype) || !float_tag(a->cs_dtype) || !float_tag(a->w_dtype) || !float_tag(a->y_dtype))
    return DFT_ERR_INVALID;
  if (a->bias && !float_tag(a->bias_dtype)) return DFT_ERR_INVALID;
  if (a->iw && !float_tag(a->iw_dtype)) return DFT_ERR_INVALID;
  if (!index_tag(a->cidx_dtype)) return DFT_ERR_INVALID;
  if (a->cs_indices && !index_tag(a->cs_indices_dtype)) return DFT_ERR_INVALID;
  if (a->iw_indices && !index_tag(a->iw_indices_dtype)) return DFT_ERR_INVALID;
  return dft::launch_tree_conv(a, static_cast<hipStream_t>(stream));
}

int dft_tree_commit(const dft_commit_args* a, void* stream) {
  if (!a) return DFT_ERR_INVALID;
  if (a->n_layers < 0 || a->batch < 0 || a->hv <= 0 || a->n_nodes < 0) return DFT_ERR_INVALID;
  if (a->dk != 128 || a->dv != 128) return DFT_ERR_UNSUPPORTED;
  if (a->path_cols < 1) return DFT_ERR_INVALID;
  if (a->n_nodes > 64 || a->path_cols > 64) return DFT_ERR_UNSUPPORTED;
  if (a->n_ends != 1 && a->n_ends != 2) return DFT_ERR_INVALID;
  if (a->k_head_div <= 0 || a->hv % a->k_head_div != 0) return DFT_ERR_INVALID;
  if (a->n_layers == 0 || a->batch == 0) return DFT_OK;
  if (!a->path || !a->keys || !a->values || !a->gains || !a->src || !a->dst) return DFT_ERR_INVALID;
  if (!index_tag(a->path_dtype)) return DFT_ERR_INVALID;
  if (a->path_len && !index_tag(a->path_len_dtype)) return DFT_ERR_INVALID;
  if (a->ends && !index_tag(a->ends_dtype)) return DFT_ERR_INVALID;
  if (a->src_slots && !index_tag(a->src_slots_dtype)) return DFT_ERR_INVALID;
  if (a->dst_slots && !index_tag(a->dst_slots_dtype)) return DFT_ERR_INVALID;
  if ((a->flags & DFT_COMMIT_CHECK_ANC) && !a->anc_bits && !a->anc_f32) return DFT_ERR_INVALID;
  // several ends writing one in-place state would race
  if (a->dst == a->src && a->n_ends != 1) return DFT_ERR_INVALID;
  const int64_t blocks = (int64_t)a->n_layers * a->batch * a->hv * a->n_ends;
  if (blocks > max_blocks(256)) return DFT_ERR_UNSUPPORTED;
  return dft::launch_tree_commit(a, static_cast<hipStream_t>(stream));
}

int dft_tree_struct(const dft_tree_args* a, void* stream) {
  if (!a) return DFT_ERR_INVALID;
  if (a->batch < 0 || a->n_nodes < 0 || a->n_nodes > 64) return DFT_ERR_INVALID;
  if (a->kc < 0 || a->kc > 16) return DFT_ERR_UNSUPPORTED;
  if (a->batch == 0) return DFT_OK;
  if (((int64_t)a->batch + 3) / 4 > max_blocks(256)) return DFT_ERR_UNSUPPORTED;  // a wave per request
  if (!a->parent || !index_tag(a->parent_dtype)) return DFT_ERR_INVALID;
  if (a->depth && !index_tag(a->depth_dtype)) return DFT_ERR_INVALID;
  if (a->cidx && (!index_tag(a->cidx_dtype) || a->kc < 1)) return DFT_ERR_INVALID;
  if ((a->nxt || a->sib) && !index_tag(a->link_dtype)) return DFT_ERR_INVALID;
  return dft::launch_tree_struct(a, static_cast<hipStream_t>(stream));
}

int dft_anc_pack(const dft_anc_pack_args* a, void* stream) {
  if (!a) return DFT_ERR_INVALID;
  if (a->batch < 0 || a->n_nodes < 0 || a->n_nodes > 64) return DFT_ERR_INVALID;
  if (a->batch == 0 || a->n_nodes == 0) return DFT_OK;
  if (((int64_t)a->batch + 3) / 4 > max_blocks(256)) return DFT_ERR_UNSUPPORTED;  // a wave per request
  if (!a->anc || !a->anc_bits) return DFT_ERR_INVALID;
  return dft::launch_anc_pack(a, static_cast<hipStream_t>(stream));
}

int dft_packbits(const dft_packbits_args* a, void* stream) {
  if (!a) return DFT_ERR_INVALID;
  if (a->bit_order != DFT_BITS_LITTLE && a->bit_order != DFT_BITS_BIG) return DFT_ERR_INVALID;
  if (a->out_capacity < 0) return DFT_ERR_INVALID;
  if (a->indptr) {
    if (a->n_segments < 0 || !index_tag(a->indptr_dtype)) return DFT_ERR_INVALID;
    if (a->n_segments > 65535) return DFT_ERR_UNSUPPORTED;
    if (a->n_segments == 0) return DFT_OK;
  } else if (a->n < 0) {
    return DFT_ERR_INVALID;
  }
  if (a->out_indptr && !index_tag(a->out_indptr_dtype)) return DFT_ERR_INVALID;
  if (!a->x || !a->out) return DFT_ERR_INVALID;
  return dft::launch_packbits(a, static_cast<hipStream_t>(stream));
}

int dft_tree_mask_pack(const dft_mask_args* a, void* stream) {
  if (!a) return DFT_ERR_INVALID;
  if (a->batch < 0 || a->n_nodes < 0 || a->n_nodes > 64) return DFT_ERR_INVALID;
  if (a->bit_order != DFT_BITS_LITTLE && a->bit_order != DFT_BITS_BIG) return DFT_ERR_INVALID;
  if (a->out_capacity < 0) return DFT_ERR_INVALID;
  if (a->batch > 65535) return DFT_ERR_UNSUPPORTED;
  if (a->batch == 0) return DFT_OK;
  if (!a->anc_bits || !a->prefix_len || !a->out || !index_tag(a->prefix_len_dtype)) return DFT_ERR_INVALID;
  if (a->out_indptr && !index_tag(a->out_indptr_dtype)) return DFT_ERR_INVALID;
  return dft::launch_tree_mask(a, static_cast<hipStream_t>(stream));
}

}  // extern "C"
