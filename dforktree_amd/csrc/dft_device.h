// Device helpers shared by the gfx950 kernels of the GDN tree-verify path.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/dforktree_amd.h"

namespace dft {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// scalar conversions and dtype-tagged loads / stores
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  // round to nearest even (inputs here are finite)
  uint32_t u = __float_as_uint(x);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float ld_f(const void* p, int64_t i, int dt) {
  switch (dt) {
    case DFT_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case DFT_F16: return __half2float(((const __half*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

__device__ __forceinline__ int64_t ld_i(const void* p, int64_t i, int dt) {
  return dt == DFT_I64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

__device__ __forceinline__ void st_f(void* p, int64_t i, int dt, float v) {
  switch (dt) {
    case DFT_BF16: ((uint16_t*)p)[i] = f32_to_bf16_bits(v); break;
    case DFT_F16: ((__half*)p)[i] = __float2half(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

__device__ __forceinline__ void st_i(void* p, int64_t i, int dt, int64_t v) {
  if (dt == DFT_I64) ((int64_t*)p)[i] = v;
  else ((int32_t*)p)[i] = (int32_t)v;
}

// bits 0..i set (the ancestor-or-self mask of a topologically ordered node i)
// a value the workgroup agrees on, as a scalar
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint64_t mask_upto(int i) {
  return i >= 63 ? ~0ull : ((1ull << (i + 1)) - 1ull);
}

__device__ __forceinline__ uint64_t mask_below(int n) {
  return n >= 64 ? ~0ull : ((1ull << n) - 1ull);
}

// ---------------------------------------------------------------------------
// MFMA wrappers (CDNA4)
// 32x32 accumulator layout: lane l, register r holds
//   row = 8*(r/4) + 4*(l/32) + r%4,  column = l%32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int acc_row(int r, int half) { return 8 * (r >> 2) + 4 * half + (r & 3); }

__device__ __forceinline__ f32x16 mfma_bf16_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// fp32 -> (hi, lo) bf16 pair with x ~= hi + lo to ~2^-17 relative
__device__ __forceinline__ void split_bf16x8(const float* x, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    f32x2 v = {x[e], x[e + 1]};
    bf16x2 h = __builtin_convertvector(v, bf16x2);
    f32x2 hf = __builtin_convertvector(h, f32x2);
    bf16x2 l = __builtin_convertvector(v - hf, bf16x2);
    hi[e] = h[0];
    hi[e + 1] = h[1];
    lo[e] = l[0];
    lo[e + 1] = l[1];
  }
}

}  // namespace dft
