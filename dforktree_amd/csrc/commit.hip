// Closed-form accepted-path state commit (tree_kernels.py:111-127 in place,
// fc1_fused.py:26-49 into a snapshot slot):
//   S_u = e^{G_u} S0 + sum_{t in path, t anc-or-self of u} e^{G_u - G_t} k_t vn_t^T
// One workgroup per (layer, request, head, end) rewrites one 128x128 fp32
// state: a rank-T update (T <= 64 accepted nodes) that is read-modify-write
// HBM traffic at ~4 flop/B, so plain fp32 FMAs from registers, the state
// streamed with 16-byte loads issued before the path bookkeeping.
//
// The state is addressed as rows x cols.  Pool layout [.., V, K] (k
// contiguous): rows = v, cols = k, so S[v][k] += (w_t vn_t[v]) k_t[k].
// With DFT_COMMIT_KV the rows are k and the update is k_t[k] (w_t vn_t[v]).
#include <initializer_list>

#include "dft_device.h"

namespace dft {

constexpr int kCD = 128;

struct CommitParams {
  dft_commit_args a;
  int src_vec, dst_vec;  // 16-byte vector path usable
};

// path entries of request b that count (path_len, or all path_cols)
__device__ __forceinline__ int path_entries(const dft_commit_args& p, int b) {
  int len = p.path_cols;
  if (p.path_len) {
    len = (int)ld_i(p.path_len, b, p.path_len_dtype);
    if (p.flags & DFT_COMMIT_LEN_IS_LAST) len += 1;
    len = len < 0 ? 0 : (len > p.path_cols ? p.path_cols : len);
  }
  return len;
}

// The status word of request b (wave 0 of its first workgroup): a row span
// past n_nodes, and path entries or ends at or past its n nodes.
__device__ __forceinline__ void commit_status(const dft_commit_args& p, int b, int n, bool span_bad, int lane) {
  const int len = path_entries(p, b);
  bool bad = false;
  for (int c = lane; c < len; c += 64) bad |= ld_i(p.path, (int64_t)b * p.path_req_stride + c, p.path_dtype) >= n;
  if (p.ends && lane < p.n_ends) bad |= ld_i(p.ends, (int64_t)b * p.ends_req_stride + lane, p.ends_dtype) >= n;
  const bool any = __ballot(bad) != 0;
  if (lane == 0) p.status[b] = (span_bad ? DFT_STATUS_SPAN : 0) | (any ? DFT_STATUS_PATH : 0);
}

// Five waves per SIMD (five workgroups per CU instead of four, 64 KiB more
// state in flight per CU): 48.3 -> 46.4 us per layer at batch 64 in
// interleaved runs.  The tile takes 64 of the 96 registers this leaves; the
// element-wise paths (layouts without 16-byte rows) walk a row pointer and
// the slot indices are scalars, so that no row index or slot is held in
// vector registers through the update and nothing is spilled.
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5)))
tree_commit_kernel(const CommitParams P) {
  const dft_commit_args& p = P.a;
  extern __shared__ float cshm[];  // rv[T][128] then cv[T][128]
  __shared__ int s_nodes[64];
  __shared__ int s_cnt, s_u;

  const int tid = threadIdx.x, lane = tid & 63;
  // block id -> (layer, request, head) unit and end.  The ends of one unit
  // read the same source tile: their blocks sit 8 ids apart, so that they
  // land on one XCD (blocks are dealt to the 8 XCDs in turn) and the later
  // reads of the tile hit that XCD's L2.  Units past the last whole group
  // of 8 take their ends from consecutive ids.
  int id = blockIdx.x, e;
  {
    const int units = p.n_layers * p.batch * p.hv;
    const int full = (units / 8) * 8 * p.n_ends;
    if (id < full) {
      const int grp = id / (8 * p.n_ends), rem = id - grp * 8 * p.n_ends;
      e = rem >> 3;
      id = grp * 8 + (rem & 7);
    } else {
      const int t = id - full;
      e = t % p.n_ends;
      id = (units / 8) * 8 + t / p.n_ends;
    }
  }
  const int h = id % p.hv;
  id /= p.hv;
  const int b = id % p.batch;
  const int l = id / p.batch;

  // nodes of the request: its row span cut to [0, n_nodes]
  int64_t row0;
  int span;
  if (p.cu_seqlens) {
    row0 = p.cu_seqlens[b];
    span = p.cu_seqlens[b + 1] - p.cu_seqlens[b];
  } else {
    row0 = (int64_t)b * p.n_nodes;
    span = p.n_nodes;
  }
  const int n = span < 0 ? 0 : (span > p.n_nodes ? p.n_nodes : span);
  if (p.status && l == 0 && h == 0 && e == 0 && tid < 64) commit_status(p, b, n, span < 0 || span > p.n_nodes, lane);

  int u_end = -1;
  if (p.ends) {
    u_end = (int)ld_i(p.ends, (int64_t)b * p.ends_req_stride + e, p.ends_dtype);
    if (u_end < 0 || u_end >= n) return;  // nothing to commit for this end
  }

  // A negative destination slot (in place: a negative source slot), e.g. a
  // padded request, commits nothing; a negative source slot with a separate
  // destination reads slot 0, as the verify reads its S0.
  int64_t slot = b;
  if (p.src_slots) slot = ld_i(p.src_slots, b, p.src_slots_dtype);
  int64_t dslot = slot;
  if (p.dst_slots) dslot = ld_i(p.dst_slots, b, p.dst_slots_dtype);
  if (dslot < 0) return;
  if (slot < 0) slot = 0;
  // uniform over the workgroup: scalar registers, not two vector ones held
  // through the update
  slot = uniform64(slot);
  dslot = uniform64(dslot);

  // ---- state tile: thread owns rows 16*rg .. 16*rg+15, cols 4*c4 .. 4*c4+3
  const int c4 = tid & 31, rg = tid >> 5;
  const float* srcp = p.src + (int64_t)l * p.src_layer_stride + slot * p.src_slot_stride + (int64_t)h * p.src_h_stride;
  f32x4 st[16];
  if (P.src_vec) {
#pragma unroll
    for (int m = 0; m < 16; ++m)
      st[m] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4*>(srcp + (int64_t)(16 * rg + m) * p.src_row_stride + 4 * c4));
  } else {  // element loads, walking the rows (no per-row index is kept live)
    const float* rowp = srcp + (int64_t)(16 * rg) * p.src_row_stride + (int64_t)(4 * c4) * p.src_col_stride;
#pragma unroll
    for (int m = 0; m < 16; ++m, rowp += p.src_row_stride)
#pragma unroll
      for (int q = 0; q < 4; ++q) st[m][q] = rowp[(int64_t)q * p.src_col_stride];
  }

  // ---- path bookkeeping on wave 0: the nodes that contribute, in path order
  if (tid < 64) {
    const int len = path_entries(p, b);
    int node = -1;
    if (lane < len) node = (int)ld_i(p.path, (int64_t)b * p.path_req_stride + lane, p.path_dtype);
    if (node >= n) node = -1;
    const bool valid = node >= 0;
    const uint64_t vmask = __ballot(valid);
    int u = u_end;
    if (!p.ends) {
      const int last = vmask ? 63 - __builtin_clzll(vmask) : 0;
      const int un = __shfl(node, last);
      u = vmask ? un : -1;
    }
    bool on = valid && u >= 0;
    if ((p.flags & DFT_COMMIT_CHECK_ANC) && u >= 0) {
      uint64_t abits;
      if (p.anc_bits) {
        abits = p.anc_bits[row0 + u];
      } else {
        const float av = lane < n ? p.anc_f32[(int64_t)b * p.anc_req_stride + (int64_t)u * p.anc_row_stride + lane] : 0.f;
        abits = __ballot(av > 0.5f);
      }
      on = on && ((abits >> (valid ? node : 0)) & 1ull);
    }
    const uint64_t onmask = __ballot(on);
    if (on) s_nodes[__builtin_popcountll(onmask & mask_below(lane))] = node;
    if (lane == 0) {
      s_cnt = __builtin_popcountll(onmask);
      s_u = u;
    }
  }
  __syncthreads();
  const int u = s_u;
  if (u < 0) return;  // no accepted node: the state stays as it is
  const int T = s_cnt;

  const float* gl = p.gains + (int64_t)l * p.g_layer_stride + (int64_t)h * p.g_h_stride;
  const float Gu = gl[(row0 + u) * p.g_row_stride];
  const float* kl = p.keys + (int64_t)l * p.k_layer_stride + (int64_t)(h / p.k_head_div) * p.k_h_stride;
  const float* vl = p.values + (int64_t)l * p.v_layer_stride + (int64_t)h * p.v_h_stride;
  const bool kv = (p.flags & DFT_COMMIT_KV) != 0;
  float* rv = cshm;
  float* cv = cshm + p.path_cols * kCD;
  for (int c = tid; c < T * kCD; c += 256) {
    const int t = c >> 7, d = c & (kCD - 1);
    const int64_t r = row0 + s_nodes[t];
    const float w = __expf(Gu - gl[r * p.g_row_stride]);
    const float kk = kl[r * p.k_row_stride + d];
    const float vv = vl[r * p.v_row_stride + d] * w;
    rv[t * kCD + d] = kv ? kk : vv;
    cv[t * kCD + d] = kv ? vv : kk;
  }
  __syncthreads();

  const float eGu = __expf(Gu);
#pragma unroll
  for (int m = 0; m < 16; ++m) st[m] *= eGu;
  for (int t = 0; t < T; ++t) {
    const f32x4 cc = *reinterpret_cast<const f32x4*>(&cv[t * kCD + 4 * c4]);
    const f32x4* rp = reinterpret_cast<const f32x4*>(&rv[t * kCD + 16 * rg]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 r = rp[q];
#pragma unroll
      for (int m = 0; m < 4; ++m) st[4 * q + m] += r[m] * cc;
    }
  }

  float* dstp = p.dst + (int64_t)l * p.dst_layer_stride + dslot * p.dst_slot_stride + (int64_t)u * p.dst_node_stride +
                (int64_t)h * p.dst_h_stride;
  if (P.dst_vec) {
#pragma unroll
    for (int m = 0; m < 16; ++m)
      __builtin_nontemporal_store(st[m], reinterpret_cast<f32x4*>(dstp + (int64_t)(16 * rg + m) * p.dst_row_stride + 4 * c4));
  } else {
    float* rowp = dstp + (int64_t)(16 * rg) * p.dst_row_stride + (int64_t)(4 * c4) * p.dst_col_stride;
#pragma unroll
    for (int m = 0; m < 16; ++m, rowp += p.dst_row_stride)
#pragma unroll
      for (int q = 0; q < 4; ++q) rowp[(int64_t)q * p.dst_col_stride] = st[m][q];
  }
}

static bool vec_ok(const float* base, int64_t col, std::initializer_list<int64_t> strides) {
  if (col != 1 || (reinterpret_cast<uintptr_t>(base) % 16) != 0) return false;
  for (int64_t s : strides)
    if (s % 4 != 0) return false;
  return true;
}

int launch_tree_commit(const dft_commit_args* a, hipStream_t stream) {
  CommitParams P;
  P.a = *a;
  P.src_vec = vec_ok(a->src, a->src_col_stride,
                     {a->src_layer_stride, a->src_slot_stride, a->src_h_stride, a->src_row_stride});
  P.dst_vec = vec_ok(a->dst, a->dst_col_stride,
                     {a->dst_layer_stride, a->dst_slot_stride, a->dst_node_stride, a->dst_h_stride,
                      a->dst_row_stride});
  const int64_t blocks = (int64_t)a->n_layers * a->batch * a->hv * a->n_ends;
  const size_t shm = (size_t)2 * a->path_cols * kCD * sizeof(float);
  hipLaunchKernelGGL(tree_commit_kernel, dim3((unsigned)blocks), dim3(256), shm, stream, P);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
