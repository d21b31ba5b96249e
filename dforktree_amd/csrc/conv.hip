// Tree-parent causal conv1d (fc1_conv.py:7-27, tree_kernels.py:17-33).
//
// For node n of request b and channel c:
//   xt[col] = col < W-1 ? conv_state[slot][c][col] : x[b][col-(W-1)][c]
//   y[b][n][c] = act(sum_j w[c][j] * xt[cidx[b][n][j]] + bias[c])
//   iw[dst][n][c][j-1] = xt[cidx[b][n][j]]            (j >= 1, optional)
// The gather columns are per node, so every thread of a block reads the
// same W indices (scalar loads) and streams channels: block = 256 channels
// x one node, loads and stores coalesced along c.  HBM-bound byte work.
#include "dft_device.h"

namespace dft {

constexpr int kMaxTaps = 8;

__global__ void __launch_bounds__(256) tree_conv_kernel(const dft_conv_args p) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  const int n = blockIdx.y, b = blockIdx.z;
  if (c >= p.channels) return;
  const int W = p.width;

  // A negative state slot (a padded request) reads slot 0; a negative window
  // slot writes no window.
  int64_t slot = b, dst = b;
  if (p.cs_indices) slot = ld_i(p.cs_indices, b, p.cs_indices_dtype);
  if (p.iw_indices) dst = ld_i(p.iw_indices, b, p.iw_indices_dtype);
  if (slot < 0) slot = 0;

  const int64_t cbase = (int64_t)b * p.cidx_req_stride + (int64_t)n * p.cidx_node_stride;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxTaps; ++j) {
    if (j >= W) break;
    const int64_t col = ld_i(p.cidx, cbase + j, p.cidx_dtype);
    float val;
    if (col < 0 || col >= W - 1 + p.n_nodes)  // outside [conv_state || x]: reads as zero
      val = 0.f;
    else if (col < W - 1)
      val = ld_f(p.conv_state, slot * p.cs_slot_stride + (int64_t)c * p.cs_chan_stride + col * p.cs_col_stride,
                 p.cs_dtype);
    else
      val = ld_f(p.x, (int64_t)b * p.x_req_stride + (col - (W - 1)) * p.x_node_stride + (int64_t)c * p.x_chan_stride,
                 p.x_dtype);
    const float w = ld_f(p.weight, (int64_t)c * p.w_chan_stride + (int64_t)j * p.w_tap_stride, p.w_dtype);
    acc += val * w;
    if (j > 0 && p.iw && dst >= 0)
      st_f(p.iw,
           dst * p.iw_slot_stride + (int64_t)n * p.iw_node_stride + (int64_t)c * p.iw_chan_stride +
               (int64_t)(j - 1) * p.iw_col_stride,
           p.iw_dtype, val);
  }
  if (p.bias) acc += ld_f(p.bias, c, p.bias_dtype);
  const float out = p.silu ? acc / (1.f + expf(-acc)) : acc;
  st_f(p.y, (int64_t)b * p.y_req_stride + (int64_t)n * p.y_node_stride + c, p.y_dtype, out);
}

// Fast path for the plugin's layout: width 4, bf16 tokens / weights / output
// / window, channel-contiguous rows.  A block of one wave (64 threads)
// covers 512 channels of one node; a thread owns 8 consecutive channels, so every
// gathered token row, the weights (8 channels x 4 taps) and the output are
// 16-byte accesses.  The gather columns are uniform over the block: the four
// come in one batch of scalar loads (the index width is a template
// parameter, so no load waits behind a dtype branch), the weights go out
// meanwhile, and the four token loads are issued unconditionally (a tap
// outside the tokens reads row 0 and is discarded).  Against a preamble of
// dependent dtype-switched index loads this measured 41.0 -> 40.5 us.
// The node's window over the block's channels is one contiguous run
// (iw[n][c][0..2]): the threads' 48-byte pieces go through LDS so that each
// store instruction writes 1 KiB of consecutive bytes (whole lines) instead
// of 16 bytes every 48.
// The grid is 1-D and XCD-aware: workgroups are dealt to the 8 XCDs round
// robin, so ids that agree mod 8 (one XCD, one L2) cover every node of one
// (request, channel block) and the parents' rows re-read by the children
// stay in that L2.
// Measured at 64 requests x 32 nodes x 8192 channels: one node per block
// beats blocks that walk 2-8 nodes (fewer, longer-lived waves) and beats
// unstaged 48-byte window stores (non-temporal unstaged stores were slower
// still: partial lines reach memory unmerged).  With the staged stores,
// non-temporal y / window stores time the same as ordinary ones (within 1%).
// Block size, in interleaved runs: one wave over 512 channels 40.0 us,
// 128 threads over 1024 channels 40.8 us, 256 threads over 2048 channels
// 41.3 us; 16 channels per thread (256 threads over 4096) 44.2 us.
// Request b's index (a slot) from an int32 or int64 array as two 32-bit
// loads with no branch between them; idx NULL reads nothing (returns 0).
__device__ __forceinline__ int64_t req_index(const void* idx, int dt, int b) {
  if (!idx) return 0;
  const int32_t* w = static_cast<const int32_t*>(idx);
  const bool wide = dt == DFT_I64;
  const int32_t lo = w[wide ? 2 * b : b];
  const int32_t hi = w[wide ? 2 * b + 1 : b];
  return wide ? (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo) : (int64_t)lo;
}

template <bool CIDX64>
__global__ void __launch_bounds__(64) tree_conv4_bf16_kernel(const dft_conv_args p, int cblocks) {
  __shared__ u32x4 stage[64 * 3];
  const int id = blockIdx.x;
  const int k = id >> 3;
  const int n = k % p.n_nodes;
  const int pair = (k / p.n_nodes) * 8 + (id & 7);
  if (pair >= p.batch * cblocks) return;  // uniform over the block
  const int cb = pair % cblocks, b = pair / cblocks;
  const int nact = min(64, (p.channels - cb * 512) / 8);  // threads with channels
  const bool active = (int)threadIdx.x < nact;
  const int c0 = (cb * 64 + threadIdx.x) * 8;

  // the node's four tap columns: independent loads, one wait
  const int64_t cbase = (int64_t)b * p.cidx_req_stride + (int64_t)n * p.cidx_node_stride;
  int64_t col[4];
  if constexpr (CIDX64) {
    const int64_t* ci = static_cast<const int64_t*>(p.cidx) + cbase;
#pragma unroll
    for (int j = 0; j < 4; ++j) col[j] = ci[j];
  } else {
    const int32_t* ci = static_cast<const int32_t*>(p.cidx) + cbase;
#pragma unroll
    for (int j = 0; j < 4; ++j) col[j] = ci[j];
  }
  // The request's conv-state slot and window slot come in the same batch:
  // read where they are used (behind a dtype branch, and the window slot
  // after the arithmetic), each was one more dependent round trip, which a
  // batch-1 launch waits out in full.  Branch-free: the index's low word, and
  // its high word for 64-bit indices (for 32-bit ones the same word again).
  const int64_t slot_raw = req_index(p.cs_indices, p.cs_indices_dtype, b);
  const int64_t dst_raw = req_index(p.iw_indices, p.iw_indices_dtype, b);
  // the weights (8 channels x 4 taps) do not depend on them
  const int cw = active ? c0 : 0;
  const u32x4* wp = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.weight) + (int64_t)cw * 4);
  uint16_t w[32];  // w[4 e + j]: channel c0 + e, tap j
#pragma unroll
  for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4*>(&w[8 * q]) = wp[q];
  int64_t slot = p.cs_indices ? slot_raw : b;
  const int64_t dst = p.iw_indices ? dst_raw : b;

  if (active) {
    const uint16_t* xb = static_cast<const uint16_t*>(p.x) + (int64_t)b * p.x_req_stride + c0;
    // the state slot (needed by conv-state taps only); a negative one reads slot 0
    if (slot < 0) slot = 0;
    // Token rows: every load is issued (a tap outside the tokens reads row 0
    // and is discarded), so none waits on a branch.  A tap on a bf16 conv-state
    // column (a node within two edges of the root) gathers the column's 8
    // values into the same registers instead, issued with the token loads:
    // read through the per-element path below (8 two-byte loads per tap, each
    // waited for in turn), these taps cost random 32-node trees about 5 us per
    // launch at batch 64 (computing a chain's columns, which reach the state
    // at 3 nodes only, ran 39.7 -> 34.7 us).
    const bool cs_bf16 = p.cs_dtype == DFT_BF16;
    u32x4 raw[4];
    bool tok[4], csg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      tok[j] = col[j] >= 3 && col[j] < 3 + p.n_nodes;
      csg[j] = cs_bf16 && col[j] >= 0 && col[j] < 3;  // uniform
      if (csg[j]) {
        const uint16_t* cs = static_cast<const uint16_t*>(p.conv_state) + slot * p.cs_slot_stride +
                             (int64_t)c0 * p.cs_chan_stride + col[j] * p.cs_col_stride;
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = cs[(int64_t)e * p.cs_chan_stride];
        raw[j] = *reinterpret_cast<const u32x4*>(h);
      } else {
        raw[j] = *reinterpret_cast<const u32x4*>(xb + (tok[j] ? col[j] - 3 : 0) * p.x_node_stride);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!tok[j] && !csg[j]) raw[j] = u32x4{0u, 0u, 0u, 0u};

    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = p.bias ? ld_f(p.bias, c0 + e, p.bias_dtype) : 0.f;
    uint16_t win[24];  // win[3 e + j - 1]
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v[8];
      if (col[j] >= 0 && col[j] < 3 && !csg[j]) {  // a conv-state column of another dtype
#pragma unroll
        for (int e = 0; e < 8; ++e)
          v[e] = ld_f(p.conv_state,
                      slot * p.cs_slot_stride + (int64_t)(c0 + e) * p.cs_chan_stride + col[j] * p.cs_col_stride,
                      p.cs_dtype);
      } else {  // a token row, a gathered bf16 state column, or zero outside [conv_state || x]
        const uint16_t* h = reinterpret_cast<const uint16_t*>(&raw[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = bf16_bits_to_f32(h[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] += v[e] * bf16_bits_to_f32(w[4 * e + j]);
        if (j > 0) win[3 * e + j - 1] = f32_to_bf16_bits(v[e]);
      }
    }
    uint16_t out[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = f32_to_bf16_bits(p.silu ? acc[e] / (1.f + expf(-acc[e])) : acc[e]);
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.y) + (int64_t)b * p.y_req_stride + (int64_t)n * p.y_node_stride +
                              c0) = *reinterpret_cast<const u32x4*>(out);
    if (p.iw) {
#pragma unroll
      for (int q = 0; q < 3; ++q) stage[threadIdx.x * 3 + q] = *reinterpret_cast<const u32x4*>(&win[8 * q]);
    }
  }
  if (p.iw) {
    __syncthreads();
    if (dst >= 0) {  // uniform over the block (one request); a negative slot writes no window
      u32x4* iw = reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.iw) + dst * p.iw_slot_stride +
                                           (int64_t)n * p.iw_node_stride + (int64_t)cb * 512 * 3);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const int i = threadIdx.x + 64 * q;
        if (i < nact * 3) iw[i] = stage[i];
      }
    }
  }
}

static bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// The fast path needs the plugin's layout; anything else takes the
// per-channel kernel above.
static bool conv4_bf16_ok(const dft_conv_args* a) {
  if (a->width != 4 || a->channels % 8) return false;
  if (a->x_dtype != DFT_BF16 || a->w_dtype != DFT_BF16 || a->y_dtype != DFT_BF16) return false;
  if (a->x_chan_stride != 1 || a->x_node_stride % 8 || a->x_req_stride % 8 || !aligned16(a->x)) return false;
  if (a->w_chan_stride != 4 || a->w_tap_stride != 1 || !aligned16(a->weight)) return false;
  if (a->y_node_stride % 8 || a->y_req_stride % 8 || !aligned16(a->y)) return false;
  if (a->iw && (a->iw_dtype != DFT_BF16 || a->iw_col_stride != 1 || a->iw_chan_stride != 3 || a->iw_node_stride % 8 ||
                a->iw_slot_stride % 8 || !aligned16(a->iw)))
    return false;
  return true;
}

int launch_tree_conv(const dft_conv_args* a, hipStream_t stream) {
  if (conv4_bf16_ok(a)) {
    const int cblocks = (a->channels + 511) / 512;
    const int64_t pairs8 = ((int64_t)a->batch * cblocks + 7) / 8;
    const dim3 grid((unsigned)(pairs8 * 8 * a->n_nodes));
    if (a->cidx_dtype == DFT_I64)
      hipLaunchKernelGGL(tree_conv4_bf16_kernel<true>, grid, dim3(64), 0, stream, *a, cblocks);
    else
      hipLaunchKernelGGL(tree_conv4_bf16_kernel<false>, grid, dim3(64), 0, stream, *a, cblocks);
  } else {
    const dim3 grid((unsigned)((a->channels + 255) / 256), (unsigned)a->n_nodes, (unsigned)a->batch);
    hipLaunchKernelGGL(tree_conv_kernel, grid, dim3(256), 0, stream, *a);
  }
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
