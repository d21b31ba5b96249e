// Tree structure from parent indices (tree_ops.py:68-89, fc1_builder.py:38-47).
// One wave per request (n <= 64 nodes, lane i = node i):
//   - ancestor-or-self set of i as a uint64 (exact closure by a parent walk;
//     the reference's five squarings stop at 31 edges, tree_ops.py:75-79),
//   - depth, conv gather columns cidx[i][kc-1-r] = kc-1 + (r-th ancestor)
//     if r <= depth else kc-1-(r-depth) (tree_ops.py:81-88),
//   - first child / next sibling links (fc1_builder.py:41-47).
// Node 0 is the root; for i >= 1 the parent is max(parent[i], 0), the clamp
// of tree_ops.py:73.  Integer work; results are bit-exact.
#include "dft_device.h"

namespace dft {

constexpr int kMaxKc = 16;

__global__ void __launch_bounds__(256) tree_struct_kernel(const dft_tree_args p) {
  __shared__ int spar[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int b = blockIdx.x * 4 + w;
  const bool active = b < p.batch;  // every wave reaches the barrier below

  int64_t row0 = 0;
  int n = 0;
  if (!active) {
  } else if (p.cu_seqlens) {
    row0 = p.cu_seqlens[b];
    n = p.cu_seqlens[b + 1] - p.cu_seqlens[b];
  } else {
    row0 = (int64_t)b * p.n_nodes;
    n = p.n_nodes;
  }
  n = n < 0 ? 0 : (n > 64 ? 64 : n);
  const int i = lane;

  int status = 0;
  int par = -1;
  if (i < n && i > 0) {
    const int64_t raw = ld_i(p.parent, row0 + i, p.parent_dtype);
    par = raw < 0 ? 0 : (int)raw;
    if (par >= n) {  // out of range: treated as a child of the root
      par = 0;
      status = 1;
    }
    if (par >= i) status = 1;  // not topologically ordered
  }
  spar[w][i] = par;
  __syncthreads();

  uint64_t bits = 0;
  int depth = 0;
  int anc_r[kMaxKc];
#pragma unroll
  for (int r = 0; r < kMaxKc; ++r) anc_r[r] = 0;
  if (i < n) {
    bits = 1ull << i;
    anc_r[0] = i;
    int cur = i, steps = 0;
    while (cur != 0 && steps < n) {
      cur = spar[w][cur];
      bits |= 1ull << cur;
      ++depth;
      ++steps;
#pragma unroll
      for (int r = 1; r < kMaxKc; ++r)
        if (r == depth) anc_r[r] = cur;
    }
    if (cur != 0) status = 2;  // cycle
  }

  if (i < n) {
    if (p.anc_bits) p.anc_bits[row0 + i] = bits;
    if (p.depth) st_i(p.depth, row0 + i, p.depth_dtype, depth);
    if (p.cidx) {
      for (int r = 0; r < p.kc && r < kMaxKc; ++r) {
        const int v = r <= depth ? (p.kc - 1 + anc_r[r]) : (p.kc - 1 - (r - depth));
        st_i(p.cidx, (row0 + i) * p.kc + (p.kc - 1 - r), p.cidx_dtype, v);
      }
    }
    if (p.nxt || p.sib) {
      int nx = -1, sb = -1;
      for (int v = n - 1; v > 0; --v)
        if (spar[w][v] == i) nx = v;
      for (int v = n - 1; v > i; --v)
        if (spar[w][v] == par) sb = v;
      if (p.nxt) st_i(p.nxt, row0 + i, p.link_dtype, nx);
      if (p.sib) st_i(p.sib, row0 + i, p.link_dtype, sb);
    }
  }
  if (!active) return;  // after the only barrier
  if (p.anc_f32) {
    // row r of the dense matrix: lane = column, coalesced
    float* base = p.anc_f32 + (int64_t)b * p.anc_req_stride;
    for (int r = 0; r < n; ++r) {
      const uint64_t rb = __shfl(bits, r);
      if (lane < n) base[(int64_t)r * p.anc_row_stride + lane] = (float)((rb >> lane) & 1ull);
    }
  }
  if (p.status) {
    const uint64_t bad1 = __ballot(status == 1), bad2 = __ballot(status == 2);
    if (lane == 0) p.status[b] = bad2 ? 2 : (bad1 ? 1 : 0);
  }
}

// Dense 0/1 ancestry rows -> the uint64 rows the verify and commit read.
// One wave per request: lane j loads column j of every row first (coalesced
// rows, all loads in flight at once), then the wave's ballot of each row is
// that row's mask; bits above the diagonal are dropped, as the kernels that
// read dense rows drop them.  Lane i keeps row i and writes it at the end.
// The loads take clamped, always valid addresses (row and column min(., n-1))
// and the ballots mask what lies outside the n x n matrix: with the bounds in
// a condition around each load, every load sat in its own branch and was
// waited for at once (batch 1: 7.4 us per launch at 32 nodes).
__global__ void __launch_bounds__(256) anc_pack_kernel(const dft_anc_pack_args p) {
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= p.batch) return;  // no barrier in this kernel
  const int n = p.n_nodes;
  if (n <= 0) return;        // (uniform) no rows
  const float* base = p.anc + (int64_t)b * p.anc_req_stride + (lane < n ? lane : n - 1);
  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) v[i] = base[(int64_t)(i < n ? i : n - 1) * p.anc_row_stride];
  const bool col_in = lane < n;
  uint64_t mine = 0;
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    const uint64_t row = i < n ? __ballot(col_in && v[i] > 0.5f) & mask_upto(i) : 0ull;
    if (lane == i) mine = row;
  }
  if (lane < n) p.anc_bits[(int64_t)b * n + lane] = mine;
}

int launch_anc_pack(const dft_anc_pack_args* a, hipStream_t stream) {
  const dim3 grid((unsigned)((a->batch + 3) / 4));
  hipLaunchKernelGGL(anc_pack_kernel, grid, dim3(256), 0, stream, *a);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

int launch_tree_struct(const dft_tree_args* a, hipStream_t stream) {
  const dim3 grid((unsigned)((a->batch + 3) / 4));
  hipLaunchKernelGGL(tree_struct_kernel, grid, dim3(256), 0, stream, *a);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
