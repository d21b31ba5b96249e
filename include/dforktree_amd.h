/*
 * dforktree_amd -- C ABI of the MI355X (gfx950) GDN tree-verify path.
 *
 * Every entry point:
 *   - takes plain device pointers, element strides and sizes in a POD
 *     descriptor plus a hipStream_t (passed as void*; NULL = legacy stream);
 *   - allocates nothing and never synchronises with the host, so it can be
 *     recorded into a hipGraph;
 *   - reads per-request slot / path indices on the device;
 *   - returns DFT_OK or a DFT_ERR_* code (dft_error_string explains it).
 *     A non-zero status means nothing was launched.
 *
 * Dtype tags (the *_dtype fields): DFT_F32, DFT_BF16, DFT_F16 for floating
 * inputs, DFT_I32 / DFT_I64 for index arrays.
 *
 * Reference interfaces replaced (Perseus037/DForkTree, dforktree/):
 *   dft_tree_verify    tree_gdn_split   tree_kernels.py:193-208 (with
 *                      _tree_prepare :135-164, invert{16,32,64}
 *                      fc1_block_inverse.py:36-83, _tree_finish :166-191) and
 *                      tree_gdn_fused   tree_kernels.py:95-108
 *   dft_tree_conv      fc1_conv.conv / install.call   fc1_conv.py:7-46 and
 *                      tree_conv_fused  tree_kernels.py:17-33, :86-93
 *   dft_tree_commit    closed_commit    tree_kernels.py:111-132 (in place) and
 *                      fc1_fused.snapshots / fused_commit fc1_fused.py:26-49,
 *                      :77-87 (snapshot into the intermediate cache)
 *   dft_tree_struct    tree_ops.tree_struct tree_ops.py:68-89 and the builder's
 *                      nxt/sib links fc1_builder.py:38-47
 *   dft_block_inverse  invert16/32/64   fc1_block_inverse.py:36-83
 *   dft_packbits       flashinfer.packbits(mask, bitorder='little') as the
 *                      attention plan override calls it, fc1_plan.py:26
 *                      (and flashinfer's segment form for batches)
 *   dft_tree_mask_pack the packed tree mask of fc1_branch64.py:39 (ones over
 *                      the prefix, Anc over the draft nodes) + fc1_plan.py:26
 */
#ifndef DFORKTREE_AMD_H
#define DFORKTREE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFT_ABI_VERSION 5

#if defined(__GNUC__)
#define DFT_API __attribute__((visibility("default")))
#else
#define DFT_API
#endif

enum dft_status {
  DFT_OK = 0,
  DFT_ERR_INVALID = 1,     /* a pointer, size, stride or alignment is invalid */
  DFT_ERR_UNSUPPORTED = 2, /* valid but not implemented here (e.g. Dk != 128) */
  DFT_ERR_LAUNCH = 3       /* the HIP runtime rejected the launch */
};

enum dft_dtype { DFT_F32 = 0, DFT_BF16 = 1, DFT_F16 = 2, DFT_I32 = 3, DFT_I64 = 4 };

/* Per-request status words (the optional `status` arrays of dft_verify_args
 * and dft_commit_args): every launch writes status[b] for every request b
 * (no clearing needed), as a set of these bits; 0 = the request was taken
 * as given. */
enum dft_request_status {
  /* the request's row span (cu_seqlens[b+1] - cu_seqlens[b]) is negative or
   * exceeds n_nodes: only its first min(span, n_nodes) rows were processed,
   * and no output row past them was written */
  DFT_STATUS_SPAN = 1,
  /* a path entry (within its length) or a commit end names a node at or past
   * the size of its tree: that entry (or end) was ignored */
  DFT_STATUS_PATH = 2,
  /* (dft_tree_commit_verify with prev_anc_bits) the valid pending entries,
   * in order, are not a walk down from the previous tree's root: some
   * entry's ancestors-or-self are not exactly the valid entries up to it
   * (an ancestor missing or out of order, a non-ancestor, a repeat).  The
   * path was not committed: the slot keeps its state, and the verify ran on
   * it. */
  DFT_STATUS_WALK = 4
};

/* ---------------------------------------------------------------------------
 * Tree verify: one fused launch of prepare + (I+A)^-1 + finish for every
 * (request, v-head).  Node i of request b lives at row row0(b)+i of y/a/b/o,
 * row0(b) = cu_seqlens[b] if cu_seqlens else b*n_nodes.
 * ------------------------------------------------------------------------- */
enum dft_verify_flags {
  DFT_VERIFY_AUX_K_PER_KHEAD = 1 /* aux_k holds one row set per k-head */
};

typedef struct dft_verify_args {
  int32_t batch;   /* requests */
  int32_t n_nodes; /* nodes per request; with cu_seqlens the maximum (longer
                      requests are cut to it: DFT_STATUS_SPAN), <= 64 */
  int32_t hk, hv;  /* q/k heads and v heads, hv % hk == 0 */
  int32_t dk, dv;  /* head dims, both 128 */
  float scale;     /* q scale (reference default dk^-0.5) */
  int32_t flags;   /* dft_verify_flags */

  /* y [rows, 2*hk*dk + hv*dv] bf16 = [q | k | v], channel stride 1 */
  const void* y;
  int64_t y_row_stride;
  const int32_t* cu_seqlens; /* [batch+1] or NULL */

  /* gate inputs a, b [rows, hv] (channel stride 1) and per-head A_log, dt_bias */
  const void* a;
  int64_t a_row_stride;
  int32_t a_dtype;
  const void* b;
  int64_t b_row_stride;
  int32_t b_dtype;
  const void* A_log;
  int32_t A_log_dtype;
  const void* dt_bias;
  int32_t dt_bias_dtype;
  const float* neg_exp_A; /* [hv] cached -exp(A_log), or NULL */

  /* tree: exactly one of anc_f32 (0/1 matrix per request) or anc_bits
   * (uint64 per row, bit j = node j is an ancestor-or-self). Nodes must be
   * in topological order (parent < child); bits above the diagonal are
   * ignored. */
  const float* anc_f32;
  int64_t anc_row_stride, anc_req_stride;
  const uint64_t* anc_bits;

  /* initial state S0(k, v) = state[slot*slot_stride + h*h_stride + k*k_stride
   * + v*v_stride], fp32.  slot = max(state_indices[b], 0), or b if NULL
   * (tree_kernels.py:184).  dft_tree_commit_verify commits nothing for a
   * request whose state index is negative. */
  const float* state;
  int64_t state_slot_stride, state_h_stride, state_k_stride, state_v_stride;
  const void* state_indices;
  int32_t state_indices_dtype;

  /* outputs o[row][h][v] (bf16 or f32), channel stride 1 */
  void* o;
  int64_t o_row_stride, o_h_stride;
  int32_t o_dtype;

  /* optional saves for the commit (fp32; NULL to skip):
   * aux_k[h'][row][dk] normalised keys (h' = h, or h/(hv/hk) with
   * DFT_VERIFY_AUX_K_PER_KHEAD), aux_v[h][row][dv] the WY values vn,
   * aux_g[h][row] the path-cumulative log decay G. */
  float* aux_k;
  int64_t aux_k_h_stride, aux_k_row_stride;
  float* aux_v;
  int64_t aux_v_h_stride, aux_v_row_stride;
  float* aux_g;
  int64_t aux_g_h_stride, aux_g_row_stride;

  /* optional [batch] dft_request_status bits (DFT_STATUS_SPAN; with
   * dft_tree_commit_verify also DFT_STATUS_PATH for the pending path) */
  int32_t* status;

  /* DFT_ABI_VERSION 4 (appended).  Optional: the packed batch's requests
   * ordered by size class, as dft_size_order writes them from the same
   * cu_seqlens and n_nodes.  A packed launch split by tree size (n_nodes >
   * 32) then gives each of its two kernels its own requests first, read from
   * the records: the workgroups past a class's count exit at the end of the
   * grid, in the slots its last generation leaves idle, instead of among the
   * work (128 requests of 8-64 nodes: 115.8 -> 113.5 us per layer).  Ignored
   * by unsplit launches; must not be written while the launch runs. */
  const int32_t* size_order;
} dft_verify_args;

DFT_API int dft_tree_verify(const dft_verify_args* args, void* stream);

/* Requests of a packed batch by size class, for dft_verify_args.size_order:
 * order[0..3] = {n_small, n_large, n_nodes, batch}, then batch records of 4 int32
 * {request, cu_seqlens[request], span, 0}: the requests of at most 32 nodes
 * (the span clamped to [0, n_nodes]) from record 0 up in request order, the
 * others from record batch - 1 down in request order.  order holds
 * 4 * (batch + 1) int32; one workgroup, no allocation.  No counterpart in the
 * reference (its launches are per tree size, tree_kernels.py:193-208): for
 * callers of packed ragged batches, once per step and shared by all layers.
 * A launch whose n_nodes or batch differs from the header's ignores the
 * records (each kernel then takes the requests in block order, as without
 * them); records written from other cu_seqlens of the same n_nodes and
 * batch are not detected here.
 * DFT_ERR_INVALID for batch < 0, n_nodes outside 1..64 or a null pointer. */
DFT_API int dft_size_order(const int32_t* cu_seqlens, int32_t batch, int32_t n_nodes, int32_t* order,
                           void* stream);

/* ---------------------------------------------------------------------------
 * Tree-parent causal conv1d: y[n,c] = act(sum_j w[c,j] xt[cidx[n,j]][c] + bias[c])
 * with xt = [conv_state columns 0..width-2 || x tokens]; optionally writes
 * the per-node window iw[dst][n][c][j-1] = xt[cidx[n,j]][c] for j >= 1.
 * ------------------------------------------------------------------------- */
typedef struct dft_conv_args {
  int32_t batch, n_nodes, channels, width; /* width = taps (<= 8) */
  int32_t silu;                            /* 1: SiLU, 0: identity */

  const void* x; /* token n of request b, channel c */
  int64_t x_req_stride, x_node_stride, x_chan_stride;
  int32_t x_dtype;

  const void* conv_state; /* [slot][c][col] */
  int64_t cs_slot_stride, cs_chan_stride, cs_col_stride;
  int32_t cs_dtype;
  const void* cs_indices; /* slot per request, or NULL: slot = b.  Negative: taps read slot 0 */
  int32_t cs_indices_dtype;

  const void* weight; /* [c][tap] */
  int64_t w_chan_stride, w_tap_stride;
  int32_t w_dtype;
  const void* bias; /* [c] or NULL */
  int32_t bias_dtype;

  const void* cidx; /* [b][n][tap] column into xt */
  int64_t cidx_req_stride, cidx_node_stride;
  int32_t cidx_dtype;

  void* y; /* [b][n][c] */
  int64_t y_req_stride, y_node_stride;
  int32_t y_dtype;

  void* iw; /* optional [dst][n][c][col] */
  int64_t iw_slot_stride, iw_node_stride, iw_chan_stride, iw_col_stride;
  int32_t iw_dtype;
  const void* iw_indices; /* dst per request, or NULL: dst = b.  Negative: no window is written */
  int32_t iw_indices_dtype;
} dft_conv_args;

DFT_API int dft_tree_conv(const dft_conv_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Closed-form accepted-path commit, for every (layer, request, head, end):
 *   S_u = e^{G_u} S0 + sum_{t in path, t anc-or-self of u} e^{G_u-G_t} k_t vn_t^T
 * written in place (dst == src, dst_node_stride 0) or into a snapshot slot.
 * The state is addressed as rows x cols with rows = v and cols = k for the
 * V-major pool layout (src_row_stride = v stride); pass DFT_COMMIT_KV to
 * address rows = k, cols = v instead.  The requests of one launch must write
 * distinct destination tiles: two requests committing into one slot race.
 * ------------------------------------------------------------------------- */
enum dft_commit_flags {
  DFT_COMMIT_KV = 1,        /* state rows are k, columns are v */
  DFT_COMMIT_CHECK_ANC = 2, /* count only path nodes that are ancestors of u */
  DFT_COMMIT_LEN_IS_LAST = 4 /* path_len holds the index of the last entry */
};

typedef struct dft_commit_args {
  int32_t n_layers, batch, hv;
  int32_t dk, dv;      /* both 128 */
  int32_t n_nodes;     /* nodes per request; with cu_seqlens the maximum (index bound), <= 64 */
  int32_t path_cols;   /* entries per request in path, 1..64 */
  int32_t n_ends;      /* 1 or 2 */
  int32_t flags;       /* dft_commit_flags */
  int32_t k_head_div;  /* aux_k head = h / k_head_div */

  const void* path; /* [b][path_cols] node ids, negative = unused */
  int64_t path_req_stride;
  int32_t path_dtype;
  const void* path_len; /* [b] number of valid entries, or NULL (all >= 0 entries) */
  int32_t path_len_dtype;
  const void* ends; /* [b][n_ends] node u to commit, negative = skip; NULL: u = last path entry */
  int64_t ends_req_stride;
  int32_t ends_dtype;

  const uint64_t* anc_bits; /* for DFT_COMMIT_CHECK_ANC: [rows] */
  const float* anc_f32;     /*   or 0/1 matrices per request */
  int64_t anc_row_stride, anc_req_stride;
  const int32_t* cu_seqlens; /* row0(b) as in dft_verify_args */

  const float* keys; /* [l][h'][row][dk] */
  int64_t k_layer_stride, k_h_stride, k_row_stride;
  const float* values; /* [l][h][row][dv] */
  int64_t v_layer_stride, v_h_stride, v_row_stride;
  const float* gains; /* [l][h][row] */
  int64_t g_layer_stride, g_h_stride, g_row_stride;

  const float* src; /* [l][slot][h][row][col] */
  int64_t src_layer_stride, src_slot_stride, src_h_stride, src_row_stride, src_col_stride;
  const void* src_slots; /* slot per request, or NULL: b.  Negative: read slot 0 (in place: nothing is written) */
  int32_t src_slots_dtype;

  float* dst; /* [l][slot][u][h][row][col] */
  int64_t dst_layer_stride, dst_slot_stride, dst_node_stride, dst_h_stride, dst_row_stride,
      dst_col_stride;
  const void* dst_slots; /* dst slot per request, or NULL: same as src slot.  Negative: nothing is written */
  int32_t dst_slots_dtype;

  /* optional [batch] dft_request_status bits: DFT_STATUS_SPAN for a row span
   * past n_nodes (nodes past n_nodes do not count), DFT_STATUS_PATH for a
   * path entry or an end at or past the request's node count */
  int32_t* status;
} dft_commit_args;

DFT_API int dft_tree_commit(const dft_commit_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Verify with the previous step's accepted path committed on the way in.
 * For every (request b, v-head h) the state tile S of slot b is read once,
 *   S <- e^{G_u} S + sum_t e^{G_u - G_t} k_t vn_t^T      (t: valid path entries)
 * with u the last valid entry (the in-place closed commit of
 * tree_kernels.py:111-127 / dft_tree_commit over the previous step's saved
 * keys, values and gains), written back to the slot, and then used as S0 of
 * the verify that `verify` describes (same fields as dft_tree_verify; the
 * state must have k stride 1 and 16-byte aligned rows).  Requests without a
 * valid entry verify on S unchanged and write nothing back.  A request with
 * no rows this step (span 0, or n_nodes 0 for the whole launch) only
 * commits: that is how a request leaving the batch (eviction, end of
 * sequence) flushes its pending path when no saves exist.  With n_nodes 0
 * the y, a, b, gate, ancestry and o fields are not read and may be NULL.
 * No counterpart in the reference: it fuses the commit that follows one
 * verify step into the next step's verify, so the state is read once per
 * layer and step instead of twice.  The previous step's keys / values / gains
 * must not alias this step's aux outputs (alternate two sets), and every
 * request's previous rows must exist in them.  The keys may also be read as
 * the previous step's raw bf16 rows (key_rows), normalised here; the verify
 * then writes no keys at all.  A slot that a request commits
 * into must not be another request's slot in the same launch (the tile is
 * updated in place while the other request would read it).
 * ------------------------------------------------------------------------- */
typedef struct dft_pending_commit {
  int32_t path_cols;    /* entries per request in path, <= 16 */
  int32_t k_head_div;   /* keys head = h / k_head_div */
  int32_t prev_n_nodes; /* previous step: rows per request (and the node-id bound) when prev_cu_seqlens is NULL */
  const void* path;     /* [b][path_cols] previous-step node ids, negative = unused */
  int64_t path_req_stride;
  int32_t path_dtype;
  const void* path_len; /* [b] entries considered, or NULL: all path_cols */
  int32_t path_len_dtype;
  const int32_t* prev_cu_seqlens; /* previous step's row0(b), or NULL: b * prev_n_nodes */

  const float* keys; /* [h'][row][dk], or NULL: key_rows below */
  int64_t k_h_stride, k_row_stride;
  const float* values; /* [h][row][dv] */
  int64_t v_h_stride, v_row_stride;
  const float* gains; /* [h][row] */
  int64_t g_h_stride, g_row_stride;
  /* DFT_ABI_VERSION 3 (appended: the fields above keep their offsets).
   * Instead of saved keys, the previous step's raw bf16 key rows: row r of
   * keys head h' = h / k_head_div at key_rows + h' kr_h_stride + r kr_row_stride
   * (elements), e.g. the k part of the previous step's y.  Each row is
   * normalised here as the verify normalises it, k / sqrt(sum k^2 + 1e-6),
   * so the verify that precedes it need not save keys (aux_k NULL).  Exactly
   * one of keys and key_rows is given; key_rows and both strides are 8-byte
   * aligned (strides multiples of 4 elements). */
  const uint16_t* key_rows;
  int64_t kr_h_stride, kr_row_stride;
  /* DFT_ABI_VERSION 3 as well.  With values NULL the commit recomputes the
   * path's values instead of reading saves: vn_t = sum_j X_tj W_j over the
   * path (X = (I + A)^-1 of the path nodes, A and W as the verify forms them,
   * W from the state the slot holds, which must be the state the previous
   * verify read).  Needs the previous step's raw bf16 value rows (row r of
   * v-head h at value_rows + h vr_h_stride + r vr_row_stride) and its b gates
   * (element (r, h) at prev_b + r pb_row_stride + h, dtype prev_b_dtype);
   * the gains are still read.  The valid entries must form a root walk of the
   * previous tree (each entry's ancestors are the valid entries before it),
   * as an accepted path does; the verify before such a commit need not save
   * values (aux_v NULL).  With both key_rows and value_rows 16-byte aligned
   * (base, and strides multiples of 8 elements, as slices of a y row are),
   * trees of up to 32 nodes take a kernel that copies the path's rows into
   * LDS ahead of the state tile (about 1% faster at batch 64); the results
   * are the same bits either way. */
  const uint16_t* value_rows;
  int64_t vr_h_stride, vr_row_stride;
  const void* prev_b;
  int64_t pb_row_stride;
  int32_t prev_b_dtype;
  /* DFT_ABI_VERSION 5 (appended).  Optional: the previous step's ancestry
   * rows (row r of the previous step's buffers, bit j = node j of its tree
   * is an ancestor-or-self, as dft_tree_struct writes them).  With them every
   * request's valid pending entries are checked to be a walk down from the
   * root (entry c's ancestors-or-self are exactly the valid entries 0..c, no
   * repeats), as fc1_fused.py:41 checks ancestry on the device; a request
   * that fails commits nothing and gets DFT_STATUS_WALK.  NULL: no check (a
   * non-walk path is then committed as given, which is wrong for a state
   * that persists). */
  const uint64_t* prev_anc_bits;
} dft_pending_commit;

DFT_API int dft_tree_commit_verify(const dft_verify_args* verify, const dft_pending_commit* pending, void* stream);

/* ---------------------------------------------------------------------------
 * Tree structure from parent indices (node 0 is the root; for i >= 1 the
 * parent is max(parent[i], 0) as tree_ops.py:73 clamps it).  Exact closure
 * for any depth.  Every output is optional.
 * ------------------------------------------------------------------------- */
typedef struct dft_tree_args {
  int32_t batch, n_nodes, kc; /* kc: conv taps for cidx (<= 16) */
  const void* parent;         /* [rows] local parent index */
  int32_t parent_dtype;
  const int32_t* cu_seqlens; /* row0(b) as in dft_verify_args */
  uint64_t* anc_bits;        /* [rows] */
  float* anc_f32;            /* [b][i][j] dense 0/1 */
  int64_t anc_row_stride, anc_req_stride;
  void* depth; /* [rows] */
  int32_t depth_dtype;
  void* cidx; /* [rows][kc] */
  int32_t cidx_dtype;
  void* nxt; /* [rows] first child or -1 */
  void* sib; /* [rows] next sibling or -1 */
  int32_t link_dtype;
  int32_t* status; /* optional [batch]: 0 ok, 1 parent not < child, 2 cycle */
} dft_tree_args;

DFT_API int dft_tree_struct(const dft_tree_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Dense ancestry to bit rows: anc_bits[b*n_nodes + i] bit j = (anc[b][i][j]
 * > 0.5) for j <= i (bits above the diagonal are dropped), n_nodes <= 64.
 * No counterpart in the reference: the plugin keeps each tree's ancestry as
 * the dense fp32 matrix that fc1_branch64.py:29 copies into
 * fc1_fused.CTX.anc once per step; packing it once lets every layer's
 * verify read 8 bytes per node instead of a dense row.
 * ------------------------------------------------------------------------- */
typedef struct dft_anc_pack_args {
  int32_t batch, n_nodes;
  const float* anc; /* [b][i][j], column stride 1 */
  int64_t anc_row_stride, anc_req_stride;
  uint64_t* anc_bits; /* [batch * n_nodes] */
} dft_anc_pack_args;

DFT_API int dft_anc_pack(const dft_anc_pack_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Bit-packed attention masks (numpy.packbits semantics).
 *
 * A segment of `bits` elements becomes ceil(bits / 8) bytes: element 8j + k
 * is bit k (DFT_BITS_LITTLE) or bit 7 - k (DFT_BITS_BIG) of byte j, any
 * non-zero element is 1, and the padding bits of the last byte are 0.
 * Segment s starts at byte out_indptr[s] = sum_{s' < s} ceil(bits_s' / 8);
 * out_indptr[segments] is the total (flashinfer's segment_packbits layout).
 * out_indptr is written when given.  Nothing is written at or past
 * out + out_capacity: bytes that do not fit are dropped and *status, when
 * given, is set to 1 (it is never cleared).
 * ------------------------------------------------------------------------- */
enum dft_bit_order { DFT_BITS_LITTLE = 0, DFT_BITS_BIG = 1 };

typedef struct dft_packbits_args {
  int32_t n_segments; /* with indptr (<= 65535); one segment without */
  int32_t bit_order;
  const uint8_t* x; /* bool / uint8 elements */
  int64_t n;        /* elements of the single segment when indptr is NULL */
  const void* indptr; /* [n_segments + 1] element offsets into x, or NULL */
  int32_t indptr_dtype;
  uint8_t* out;
  int64_t out_capacity; /* bytes */
  void* out_indptr;     /* [segments + 1] byte offsets, or NULL */
  int32_t out_indptr_dtype;
  int32_t* status; /* optional */
} dft_packbits_args;

DFT_API int dft_packbits(const dft_packbits_args* args, void* stream);

/* The packed tree mask without a boolean mask in between.  Request b with
 * n_b nodes (rows row0(b) .. row0(b) + n_b - 1, row0 as in dft_verify_args,
 * n_b <= 64) and plen_b committed prefix tokens is one segment: the
 * row-major n_b x (plen_b + n_b) matrix
 *   M[i][p] = p < plen_b  ||  bit (p - plen_b) of anc_bits[row0(b) + i]
 * (anc_bits as dft_tree_struct writes them: ancestor-or-self). */
typedef struct dft_mask_args {
  int32_t batch, n_nodes; /* n_nodes: nodes per request without cu_seqlens */
  int32_t bit_order;
  const int32_t* cu_seqlens;
  const uint64_t* anc_bits; /* [rows] */
  const void* prefix_len;   /* [batch] */
  int32_t prefix_len_dtype;
  uint8_t* out;
  int64_t out_capacity;
  void* out_indptr; /* [batch + 1] byte offsets, or NULL */
  int32_t out_indptr_dtype;
  int32_t* status; /* optional */
} dft_mask_args;

DFT_API int dft_tree_mask_pack(const dft_mask_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * In-place (I + A)^-1 of n_mats strictly-lower-triangular fp32 n x n matrices
 * (n <= 64, row-major, consecutive matrices mat_stride elements apart).
 * The upper triangle of the result is zeroed.
 * ------------------------------------------------------------------------- */
DFT_API int dft_block_inverse(float* x, int32_t n_mats, int32_t n, int64_t mat_stride, void* stream);

DFT_API const char* dft_error_string(int status);
DFT_API int dft_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DFORKTREE_AMD_H */
