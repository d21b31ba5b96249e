// Bit-packed attention masks for the attention layers' tree verify:
//   dft_packbits        flashinfer.packbits / segment_packbits as
//                       fc1_plan.py:26 calls it (numpy.packbits semantics)
//   dft_tree_mask_pack  the packed tree mask itself: fc1_branch64.py:39
//                       builds [ones(n, plen) | Anc] row-major and
//                       fc1_plan.py:26 packs it; here it is built straight
//                       from the ancestry bits, with no boolean mask.
//
// Both are HBM-bound byte work.  A segment (one packbits segment, one
// request's mask) starts at the byte offset sum_{s' < s} ceil(bits_s' / 8);
// every workgroup of a segment computes that sum itself (a block reduction
// over the earlier segments' sizes), so one launch suffices and nothing is
// read back by the host.  A thread produces one 32-bit word of its
// segment's bit stream (bit t of the word = element 32w + t) and stores its
// bytes.
#include <stdint.h>

#include "dft_device.h"

namespace dft {
namespace {

constexpr int kThreads = 256;
constexpr int kBlocksPerSegment = 8;  // workgroups per segment (grid-stride over its words)

__device__ __forceinline__ uint32_t low_mask(int bits) { return bits >= 32 ? 0xffffffffu : ((1u << bits) - 1u); }

// little order: element 8j + k -> bit k of byte j; big: bit 7 - k
__device__ __forceinline__ uint32_t to_order(uint32_t w, int order) {
  return order == DFT_BITS_BIG ? __builtin_bswap32(__builtin_bitreverse32(w)) : w;
}

// Sum over threads of a block (int64); every thread gets the total.
__device__ __forceinline__ int64_t block_sum(int64_t v, int64_t* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int64_t t = 0;
  for (int i = 0; i < kThreads / 64; ++i) t += red[i];
  __syncthreads();
  return t;
}

// Store the bytes of word w of a segment that starts at byte `off` and has
// `nbytes` bytes; nothing at or past `cap`.  Returns false if a byte of the
// segment was dropped.
__device__ __forceinline__ bool store_word(uint8_t* out, int64_t cap, int64_t off, int64_t nbytes, int64_t w,
                                           uint32_t word) {
  const int64_t at = off + 4 * w;
  if ((reinterpret_cast<uintptr_t>(out + at) & 3) == 0 && 4 * w + 4 <= nbytes && at + 4 <= cap) {  // aligned word
    *reinterpret_cast<uint32_t*>(out + at) = word;
    return true;
  }
  bool ok = true;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t j = 4 * w + b;
    if (j < nbytes) {
      if (off + j < cap)
        out[off + j] = (uint8_t)(word >> (8 * b));
      else
        ok = false;
    }
  }
  return ok;
}

__device__ __forceinline__ void store_indptr(void* p, int dt, int64_t i, int64_t v) {
  if (dt == DFT_I64)
    static_cast<int64_t*>(p)[i] = v;
  else
    static_cast<int32_t*>(p)[i] = (int32_t)v;
}

// ---- generic packbits ------------------------------------------------------
__device__ __forceinline__ int64_t seg_begin(const dft_packbits_args& a, int s) {
  return a.indptr ? ld_i(a.indptr, s, a.indptr_dtype) : 0;
}
__device__ __forceinline__ int64_t seg_len(const dft_packbits_args& a, int s) {
  if (!a.indptr) return a.n;
  const int64_t l = ld_i(a.indptr, s + 1, a.indptr_dtype) - ld_i(a.indptr, s, a.indptr_dtype);
  return l < 0 ? 0 : l;
}

__global__ void __launch_bounds__(kThreads) packbits_kernel(const dft_packbits_args a) {
  __shared__ int64_t red[kThreads / 64];
  const int s = blockIdx.y;
  int64_t part = 0;
  for (int q = threadIdx.x; q < s; q += kThreads) part += (seg_len(a, q) + 7) >> 3;
  const int64_t off = block_sum(part, red);
  const int64_t len = seg_len(a, s), nbytes = (len + 7) >> 3, nwords = (len + 31) >> 5;
  if (a.out_indptr && blockIdx.x == 0 && threadIdx.x == 0) {
    store_indptr(a.out_indptr, a.out_indptr_dtype, s, off);
    if (s + 1 == (int)gridDim.y) store_indptr(a.out_indptr, a.out_indptr_dtype, s + 1, off + nbytes);
  }
  const uint8_t* x = a.x + seg_begin(a, s);
  bool ok = true;
  for (int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x; w < nwords; w += (int64_t)gridDim.x * kThreads) {
    uint32_t word = 0;
    const int64_t e0 = 32 * w;
#pragma unroll 8
    for (int t = 0; t < 32; ++t)
      if (e0 + t < len && x[e0 + t] != 0) word |= 1u << t;
    ok &= store_word(a.out, a.out_capacity, off, nbytes, w, to_order(word, a.bit_order));
  }
  if (!ok && a.status) *a.status = 1;
}

// ---- packed tree mask -------------------------------------------------------
struct MaskSeg {
  int64_t row0;  // row of node 0
  int64_t plen;  // committed prefix tokens
  int n;         // nodes (<= 64)
};

__device__ __forceinline__ MaskSeg mask_seg(const dft_mask_args& a, int b) {
  MaskSeg m;
  if (a.cu_seqlens) {
    m.row0 = a.cu_seqlens[b];
    m.n = a.cu_seqlens[b + 1] - a.cu_seqlens[b];
  } else {
    m.row0 = (int64_t)b * a.n_nodes;
    m.n = a.n_nodes;
  }
  m.n = m.n < 0 ? 0 : (m.n > 64 ? 64 : m.n);
  const int64_t pl = ld_i(a.prefix_len, b, a.prefix_len_dtype);
  m.plen = pl < 0 ? 0 : pl;
  return m;
}

__device__ __forceinline__ int64_t mask_bits(const MaskSeg& m) { return (int64_t)m.n * (m.plen + m.n); }

// columns c .. c + take - 1 (take <= 32, within one row) of the row whose
// ancestor-or-self bits are `anc`: ones below plen, then the ancestry bits
__device__ __forceinline__ uint32_t row_bits(uint64_t anc, int64_t plen, int64_t c, int take) {
  if (c + take <= plen) return low_mask(take);
  if (c >= plen) return (uint32_t)(anc >> (c - plen)) & low_mask(take);  // c - plen < n <= 64
  const int k = (int)(plen - c);                                          // 1 .. take - 1
  return low_mask(k) | ((uint32_t)(anc << k) & low_mask(take));
}

__global__ void __launch_bounds__(kThreads) tree_mask_kernel(const dft_mask_args a) {
  __shared__ int64_t red[kThreads / 64];
  const int b = blockIdx.y;
  int64_t part = 0;
  for (int q = threadIdx.x; q < b; q += kThreads) part += (mask_bits(mask_seg(a, q)) + 7) >> 3;
  const int64_t off = block_sum(part, red);
  const MaskSeg m = mask_seg(a, b);
  const int64_t L = m.plen + m.n, nbits = mask_bits(m), nbytes = (nbits + 7) >> 3, nwords = (nbits + 31) >> 5;
  if (a.out_indptr && blockIdx.x == 0 && threadIdx.x == 0) {
    store_indptr(a.out_indptr, a.out_indptr_dtype, b, off);
    if (b + 1 == (int)gridDim.y) store_indptr(a.out_indptr, a.out_indptr_dtype, b + 1, off + nbytes);
  }
  bool ok = true;
  for (int64_t w = (int64_t)blockIdx.x * kThreads + threadIdx.x; w < nwords; w += (int64_t)gridDim.x * kThreads) {
    const int64_t q0 = 32 * w;
    int64_t r, c;
    if (nbits <= 0x7fffffff) {  // 32-bit division (uniform per request)
      r = (uint32_t)q0 / (uint32_t)L;
      c = q0 - r * L;
    } else {
      r = q0 / L;
      c = q0 - r * L;
    }
    uint32_t word = 0;
    int done = 0;
    while (done < 32 && r < m.n) {  // at most 32 rows (rows are >= 1 bit long)
      const int take = (int)(L - c < 32 - done ? L - c : 32 - done);
      word |= row_bits(a.anc_bits[m.row0 + r], m.plen, c, take) << done;
      done += take;
      ++r;
      c = 0;
    }
    ok &= store_word(a.out, a.out_capacity, off, nbytes, w, to_order(word, a.bit_order));
  }
  if (!ok && a.status) *a.status = 1;
}

}  // namespace

int launch_packbits(const dft_packbits_args* a, hipStream_t stream) {
  const int segs = a->indptr ? a->n_segments : 1;
  // one segment of known length: enough workgroups to cover it once
  int bx = kBlocksPerSegment;
  if (!a->indptr) {
    const int64_t words = (a->n + 31) >> 5, need = (words + kThreads - 1) / kThreads;
    bx = (int)(need < 1 ? 1 : (need > 4096 ? 4096 : need));
  }
  hipLaunchKernelGGL(packbits_kernel, dim3((unsigned)bx, (unsigned)segs), dim3(kThreads), 0, stream, *a);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

int launch_tree_mask(const dft_mask_args* a, hipStream_t stream) {
  hipLaunchKernelGGL(tree_mask_kernel, dim3(kBlocksPerSegment, (unsigned)a->batch), dim3(kThreads), 0, stream, *a);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
