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

  int64_t slot = b, dst = b;
  if (p.cs_indices) slot = ld_i(p.cs_indices, b, p.cs_indices_dtype);
  if (p.iw_indices) dst = ld_i(p.iw_indices, b, p.iw_indices_dtype);

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
    if (j > 0 && p.iw)
      st_f(p.iw,
           dst * p.iw_slot_stride + (int64_t)n * p.iw_node_stride + (int64_t)c * p.iw_chan_stride +
               (int64_t)(j - 1) * p.iw_col_stride,
           p.iw_dtype, val);
  }
  if (p.bias) acc += ld_f(p.bias, c, p.bias_dtype);
  const float out = p.silu ? acc / (1.f + expf(-acc)) : acc;
  st_f(p.y, (int64_t)b * p.y_req_stride + (int64_t)n * p.y_node_stride + c, p.y_dtype, out);
}

int launch_tree_conv(const dft_conv_args* a, hipStream_t stream) {
  const dim3 grid((unsigned)((a->channels + 255) / 256), (unsigned)a->n_nodes, (unsigned)a->batch);
  hipLaunchKernelGGL(tree_conv_kernel, grid, dim3(256), 0, stream, *a);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
