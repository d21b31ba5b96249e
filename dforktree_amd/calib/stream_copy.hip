// Streaming device copy: the achievable-bandwidth reference that bench.py
// reports beside the 8 TB/s HBM peak.  Not part of the tree-verify path or
// its C ABI; built into its own library (libdft_stream_copy.so).
//
// One 16-byte non-temporal load and store per thread, 256 threads per
// workgroup, one workgroup per 4 KiB.  On MI355X this form outruns the
// unrolled and grid-stride variants and the runtime's device-to-device copy.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_copy_kernel(const f4* __restrict__ src, f4* __restrict__ dst,
                                                          int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Copies `bytes` (a positive multiple of 16; both pointers 16-byte aligned)
// on `stream`.  Returns 0, 1 for invalid arguments, 2 for a launch error.
extern "C" __attribute__((visibility("default"))) int dft_calib_stream_copy(const void* src, void* dst,
                                                                             int64_t bytes, void* stream) {
  if (src == nullptr || dst == nullptr || bytes <= 0 || (bytes & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(src) & 15) != 0 || (reinterpret_cast<uintptr_t>(dst) & 15) != 0)
    return 1;
  const int64_t n16 = bytes / 16;
  const int64_t grid = (n16 + 255) / 256;
  if (grid > 0x7fffffff) return 1;
  stream_copy_kernel<<<dim3((unsigned)grid), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const f4*>(src), static_cast<f4*>(dst), n16);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
