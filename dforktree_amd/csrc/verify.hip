// Fused GDN tree verify for gfx950: one workgroup per (request, v-head)
// (4 wave64 for trees of up to 32 nodes, 8 for 33-64) does prepare +
// (I+A)^-1 + finish of tree_kernels.py:135-208 in a single pass over the
// recurrent state.
//
// Math (per head; q_n = rq q_raw, k_n = rk k_raw with q_raw/k_raw the exact
// bf16 rows, so every MFMA left operand on the state is exact):
//   G_i   = sum_{j anc-or-self i} g_j
//   A_ij  = [j strict anc i] beta_i (k_n,i . k_n,j) e^{G_i - G_j}
//   Pq_ij = [j anc-or-self i] (q_n,i . k_n,j) e^{G_i - G_j}
//   X     = (I + A)^-1
//   Cq    = q_raw S0,  Ck = k_raw S0                   (bf16 MFMA, S0 split hi+lo)
//   W     = diag(beta) (v - diag(e^G rk) Ck)
//   vn    = X W  (= X(beta v) - X(beta e^G k) S0 of :182-186)
//   o     = diag(e^G rq) Cq + Pq vn  (= (e^G q) S0 + Pq vn of :190)
//
// Phases:
//  0. the 64 KiB state tile streams straight into MFMA B operands of
//     v_mfma_f32_16x16x32_bf16 (lane (n = l%16, g = l/16) loads 16 bytes at
//     k = 16j + 4g of state row n: the 4 lanes of a row cover a 64-byte
//     sector per instruction); q/k/v rows, gates and ancestry go to LDS.
//     The verify issues the tile in four k-step groups spread over phase 1;
//     the 64-wide form copies its v rows only after Cq (LDS budget).
//  1. while the state is in flight: norms, G, the Gram tiles of A, the
//     blocked inverse X (16x16 diagonal blocks by forward substitution,
//     off-diagonal blocks X_ij = -D_i sum_m A_im X_mj by fp32 MFMA), then
//     the masked, scaled Gram Pq into the LDS that A held; X and Pq are kept
//     as bf16 hi/lo operand pairs from here on (split once, not per wave).
//  2. Cq, Ck on the wave's value columns.
//  3. vn = X W, then o = cO Cq + Pq vn (o = cO Cq + M W with M = Pq X, whose
//     N^3 product is never formed), each a bf16x3 MFMA product (hi*hi +
//     hi*lo + lo*hi) whose A operand is the right factor in the accumulator
//     layout of phase 2, read with the node permutation that layout implies;
//     the products come out transposed, so vn and o leave through LDS as
//     whole row pieces.
// Every wave streams its own columns of the state; LDS holds the q/k/v rows
// and the per-head O(N^2) arrays.  The fused commit -> verify form commits
// the previous step's accepted path into the tile and writes it back: the
// 64-wide form as soon as the tile has landed, before the Gram phase; the
// 32-wide form after phase 1 (which needs no state), so that phase 1 runs
// under the state stream and only phases 2-3 follow the write-back.
#include <climits>
#include <type_traits>

#include "dft_device.h"

namespace dft {

constexpr int kD = 128;

// Waves per workgroup: 4 for trees of up to 32 nodes, 8 for 33-64 (WavesFor).
// Wave w owns value columns CW w .. CW w + CW - 1 (CW = 128 / NW), as TT = CW / 16
// MFMA column tiles; phase 1 spreads its tiles and blocks over all NW waves.
template <int NW>
struct Waves {
  static constexpr int NT = 64 * NW;  // threads
  static constexpr int CW = kD / NW;  // value columns per wave
  static constexpr int TT = CW / 16;  // 16-column tiles per wave
};
template <int NP>
constexpr int WavesFor() { return NP > 32 ? 8 : 4; }
// q/k/v rows in LDS: 256-byte rows of 16 chunks of 8 bf16, chunk c of row i
// stored at position c ^ (i & 15).  The swizzle keeps the column reads of
// 16 consecutive rows on distinct banks without padding, so a row group is
// one contiguous 1 KiB block that a single global->LDS load fills.
__device__ __forceinline__ int qkv_at(int i, int c) { return i * kD + ((((c >> 3) ^ i) & 15) << 3) + (c & 7); }
// The MFMA operand reads of these rows, lane (n, g) at row 16mt + n, with the
// swizzle's lane part computed once: row 16mt + n adds the constant 16mt kD,
// and k-step s (columns + 32s) flips chunk bits 2-3, i.e. offset ^ 32s.
//   qkv_op8(n, g):  columns 8g .. + 7          (qkv_at(16mt + n, 32s + 8g) = 16mt kD + (off ^ 32s))
//   qkv_op4(n, g):  columns 4g .. + 3, and at off ^ 16 columns 16 + 4g .. + 3
__device__ __forceinline__ int qkv_op8(int n16, int g4) { return (n16 * kD) | (((g4 ^ n16) & 15) << 3); }
__device__ __forceinline__ int qkv_op4(int n16, int g4) {
  return (n16 * kD) | (4 * (g4 & 1)) | ((((g4 >> 1) ^ n16) & 15) << 3);
}

// s_waitcnt immediate (gfx9 encoding): wait until at most vm vector-memory
// and lgkm LDS/scalar operations of this wave are outstanding
constexpr unsigned waitcnt_imm(int vm, int lgkm) {
  return (unsigned)((vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8));
}

// The aligned 32-bit word holding element i of a float tensor (F32, BF16 or
// F16), and the shift of the element within it (16 for the upper half of a
// 16-bit pair).  The word never leaves the element's page.
__device__ __forceinline__ const uint32_t* word_of(const void* p, int64_t i, int dt, uint32_t& sh) {
  const char* base = static_cast<const char*>(p);
  const int mis = (int)(reinterpret_cast<uintptr_t>(base) & 3);
  const int64_t off = i * (dt == DFT_F32 ? 4 : 2) + mis;
  sh = (uint32_t)(off & 2) << 3;
  return reinterpret_cast<const uint32_t*>(base + ((off & ~(int64_t)3) - mis));
}
__device__ __forceinline__ float word_to_f(uint32_t w, uint32_t sh, int dt) {
  if (dt == DFT_F32) return __uint_as_float(w);
  const uint32_t h = (w >> sh) & 0xffffu;
  if (dt == DFT_BF16) return __uint_as_float(h << 16);
  return __half2float(__ushort_as_half((unsigned short)h));
}

// global -> LDS copies that bypass registers: lane l's bytes land at
// lds + l * size
__device__ __forceinline__ void lds_dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
// the same with the non-temporal cache policy (data read once)
__device__ __forceinline__ void lds_dma16_nt(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 2);
}
// lds_dma16_nt issued from inline assembly, which the backend's wait
// analysis does not see.  For the late v rows it cannot tell the copy's LDS
// destination (the q rows' region) from the k rows read next and would wait
// for the copy at once; the caller waits (vmcnt) before the destination is
// read.  An untracked load issued before a tracked one leaves the backend's
// own counted waits exact (vector memory returns in issue order); issued
// after, it only makes them wait longer.  Measured at 64 nodes: 2.1% faster.
__device__ __forceinline__ void lds_dma16_nt_untracked(const void* g, void* lds) {
  const uint32_t base =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  // m0 is reserved to the backend: its value is kept across the statement.
  // A DMA needs one wait state after m0 is written (s_nop 0), and so does a
  // DMA of the backend's own right after the restore.
  uint32_t keep;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0"
      : "=&s"(keep)
      : "v"(g), "s"(base)
      : "memory");
}
__device__ __forceinline__ void lds_dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}
// a 4-byte copy the backend's wait analysis does not see (as
// lds_dma16_nt_untracked); the caller makes sure it has landed before the
// destination is read
__device__ __forceinline__ void lds_dma4_untracked(const void* g, void* lds) {
  const uint32_t base =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds);
  uint32_t keep;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0"
      : "=&s"(keep)
      : "v"(g), "s"(base)
      : "memory");
}

struct VerifyParams {
  dft_verify_args a;
  dft_pending_commit c;  // the fused commit -> verify form only
  int s0_vec;    // state rows 16-byte aligned with k stride 1 (selects the kernel)
  int auxk_vec;  // aux_k rows 16-byte aligned
  int vn_stage;  // vn rows 16-byte aligned: written as whole rows through LDS
  int o_stage;   // o is bf16 with 16-byte aligned head rows: written through LDS
  int n_lo, n_hi;  // packed launches split by tree size: this kernel takes the
                   // requests with n_lo <= nodes <= n_hi (the others exit at once)
  int cls;         // with a.size_order: this kernel's size class (0: at most 32
                   // nodes, 1: more), its requests read from the order records; -1: none
};

// The output fields a workgroup needs only at the end of its life (the key
// and gain saves, the staged vn and o stores).  The compiler loads kernel
// arguments at entry; in the fused commit -> verify kernels, whose
// registers are full, these would stay live through the whole workgroup and
// be spilled (36 scalar registers, 284 lane reads).  There they are re-read
// from the kernel-argument segment where they are used instead, through a
// pointer the compiler cannot equate with the entry loads: fused kernel
// 83.0 -> 82.0 us at batch 64.  (The verify kernels do not spill; reading
// late there only adds latency.)
struct OutArgs {
  float* aux_k;
  int64_t aux_k_h_stride, aux_k_row_stride;
  float* aux_v;
  int64_t aux_v_h_stride, aux_v_row_stride;
  float* aux_g;
  int64_t aux_g_h_stride, aux_g_row_stride;
  void* o;
  int64_t o_row_stride, o_h_stride;
  int32_t flags;
  int auxk_vec, vn_stage, o_stage;
};

template <class PP>
__device__ __forceinline__ OutArgs out_args_of(PP P) {
  OutArgs r;
  r.aux_k = P->a.aux_k;
  r.aux_k_h_stride = P->a.aux_k_h_stride;
  r.aux_k_row_stride = P->a.aux_k_row_stride;
  r.aux_v = P->a.aux_v;
  r.aux_v_h_stride = P->a.aux_v_h_stride;
  r.aux_v_row_stride = P->a.aux_v_row_stride;
  r.aux_g = P->a.aux_g;
  r.aux_g_h_stride = P->a.aux_g_h_stride;
  r.aux_g_row_stride = P->a.aux_g_row_stride;
  r.o = P->a.o;
  r.o_row_stride = P->a.o_row_stride;
  r.o_h_stride = P->a.o_h_stride;
  r.flags = P->a.flags;
  r.auxk_vec = P->auxk_vec;
  r.vn_stage = P->vn_stage;
  r.o_stage = P->o_stage;
  return r;
}

template <bool LATE>
__device__ __forceinline__ OutArgs out_args(const VerifyParams& P) {
  if constexpr (LATE) {
    // the kernel's only argument is the VerifyParams, at offset 0
    typedef const __attribute__((address_space(4))) VerifyParams* KParams;
    KParams kp = (KParams)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kp));
    return out_args_of(kp);
  } else {
    return out_args_of(&P);
  }
}

// Output staging in the (then free) q/k/v region: vn as NP x 128 fp32 with
// 16-byte chunk q of row i at q ^ (i & 31), o as NP x 128 bf16 with the
// q/k/v swizzle; both keep the accumulator-layout writes conflict-free.
__device__ __forceinline__ int vn_at(int i, int c) { return i * kD + ((((c >> 2) ^ i) & 31) << 2) + (c & 3); }

// LDS of the fused commit -> verify form: the previous step's path keys,
// 16 rows of 128 fp32 with 16-byte chunk q of row p at q ^ ((p & 3) << 2),
// so the MFMA operand reads of 4 rows x 16 columns hit 64 distinct banks.
__device__ __forceinline__ int pkey_at(int p, int c) { return p * kD + ((((c >> 2) ^ ((p & 3) << 2)) & 31) << 2) + (c & 3); }

// The 64-wide fused commit stages the previous step's 16 path keys (16 x 128
// floats) in am + x before the Gram tiles are formed; the two arrays are
// adjacent.  The 32-wide one stages them, and then its write-back, in the v
// region (exactly 16 x 128 floats), before the v rows are copied in.
//
// Trees of 33-64 nodes (NP = 64) keep no v region: their v rows are copied
// into the q region once Cq/Ck have consumed it, and o is staged in x once the
// vn tiles have consumed X.  That keeps the workgroup under 80 KiB of LDS, so
// two of them fit on a CU.
template <int NP, bool LATE_V>
struct VRegion {
  uint16_t v[NP * kD];
};
template <int NP>
struct VRegion<NP, true> {};

template <int NP>
struct VerifySmem : VRegion<NP, (NP > 32)> {
  static constexpr int LDA = NP + 4;  // fp32 row pitch, rows 16-byte aligned
  static constexpr bool kLateV = NP > 32;
  uint16_t q[NP * kD], k[NP * kD];
  // am (at[m][i] = A[i][m] until X is formed, then Pq[i][j]) and x (X[i][j]),
  // one array so that the 16 staged path keys can span both; Pq and, once
  // every level is formed, X are held in the split operand layout of phase_pq
  // (the same 4 bytes per element)
  alignas(16) float amx[2 * NP * LDA];
  // per-node arrays, 16-byte aligned: the tile epilogues read 4 consecutive nodes at once
  alignas(16) float gc[NP];  // g, then e^G rk once G is formed
  alignas(16) float G[NP];
  alignas(16) float beta[NP];
  alignas(16) float rq[NP];
  alignas(16) float rk[NP];
  alignas(16) float cO[NP];
  alignas(16) uint64_t anc[NP];
  uint32_t graw[6][64];  // per lane of wave 0: words of a, b, ancestry bits lo / hi, dt_bias, decay
  __device__ float* am() { return amx; }
  __device__ const float* am() const { return amx; }
  __device__ float* x() { return amx + NP * LDA; }
  __device__ const float* x() const { return amx + NP * LDA; }
  __device__ float* pkey() { return amx; }
  // where the v rows are read and where o is staged
  __device__ uint16_t* vrows() {
    if constexpr (kLateV) return q; else return this->v;
  }
  __device__ const uint16_t* vrows() const {
    if constexpr (kLateV) return q; else return this->v;
  }
  __device__ uint16_t* ostage() {
    if constexpr (kLateV) return reinterpret_cast<uint16_t*>(x()); else return this->v;
  }
  __device__ const uint16_t* ostage() const {
    if constexpr (kLateV) return reinterpret_cast<const uint16_t*>(x()); else return this->v;
  }
};
static_assert(sizeof(VerifySmem<64>) <= 80 * 1024, "two 64-wide workgroups per CU");
static_assert(2 * 32 * 36 >= 16 * kD && 2 * 64 * 68 >= 16 * kD, "am + x hold the 16 staged path keys");
static_assert(2 * 32 * 36 >= 4 * 512 && 2 * 64 * 68 >= 8 * 512, "am + x hold every wave's 2 KiB write-back staging");

// The mixed-width kernel's LDS (tree_verify_mixed_kernel): one 64-wide item's
// arrays, or two 32-wide items' side by side.  Only that kernel touches it.
constexpr int kMixedLds = sizeof(VerifySmem<64>) > 2 * sizeof(VerifySmem<32>) ? (int)sizeof(VerifySmem<64>)
                                                                              : (int)(2 * sizeof(VerifySmem<32>));
static_assert(sizeof(VerifySmem<32>) % 16 == 0 && kMixedLds <= 80 * 1024, "two mixed workgroups per CU");
__shared__ uint4 mixed_lds[kMixedLds / 16];

__device__ __forceinline__ f32x4 mfma_bf16_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Forward substitution on one 32-node block held in registers:
// x[i] -= A[base+i][base+m] x[m] for m < i (at[m][i] = A[i][m], pitch LDA).
template <int LDA>
__device__ __forceinline__ void solve_block32(float (&x)[32], const float* at, int base) {
#pragma unroll
  for (int m = 0; m < 31; ++m) {
    const float xm = x[m];
#pragma unroll
    for (int i = m + 1; i < 32; ++i) x[i] -= at[(base + m) * LDA + base + i] * xm;
  }
}

// y[i] -= sum_m A[ib+i][mb+m] x[m] (an off-diagonal 32x32 block)
template <int LDA>
__device__ __forceinline__ void update_block32(float (&y)[32], const float (&x)[32], const float* at, int mb, int ib) {
#pragma unroll
  for (int m = 0; m < 32; ++m) {
    const float xm = x[m];
#pragma unroll
    for (int i = 0; i < 32; ++i) y[i] -= at[(mb + m) * LDA + ib + i] * xm;
  }
}

// Forces x to be computed here: without a use at this point the compiler may
// sink pure register arithmetic below a following barrier while the loads it
// consumes stay above it, leaving every loaded operand live at once.
__device__ __forceinline__ void materialize32(const float (&x)[32]) {
#pragma unroll
  for (int i = 0; i < 32; i += 8)
    asm volatile("" ::"v"(x[i]), "v"(x[i + 1]), "v"(x[i + 2]), "v"(x[i + 3]), "v"(x[i + 4]), "v"(x[i + 5]),
                 "v"(x[i + 6]), "v"(x[i + 7]));
}

// 8 bf16 as two 8-byte halves (columns c0..c0+3 and c0+16..c0+19 of a row)
__device__ __forceinline__ bf16x8 lds_bf16x8_split(const uint16_t* first, const uint16_t* second) {
  const uint2 lo = *reinterpret_cast<const uint2*>(first);
  const uint2 hi = *reinterpret_cast<const uint2*>(second);
  const uint4 w = {lo.x, lo.y, hi.x, hi.y};
  return __builtin_bit_cast(bf16x8, w);
}

// 8 fp32 of one LDS row at columns c0..c0+3 and c0+16..c0+19
__device__ __forceinline__ void lds_f32x8_split(const float* row, int c0, float (&out)[8]) {
  const f32x4 lo = *reinterpret_cast<const f32x4*>(row + c0);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(row + c0 + 16);
  out[0] = lo[0]; out[1] = lo[1]; out[2] = lo[2]; out[3] = lo[3];
  out[4] = hi[0]; out[5] = hi[1]; out[6] = hi[2]; out[7] = hi[3];
}

// Forward substitution on one 16x16 unit-lower block: x <- (I + A_bb)^-1 e_j.
// Step m reads row m of at (A's column m) from column m + 1 on; the rows are
// 16-byte aligned (LDA and base multiples of 4), so a step's values come as
// whole 16-byte reads (from the chunk holding column m + 1), issued kAhead
// steps before their use.  Read element by element, each step's values came
// as 4- and 8-byte reads, each followed by a wait: at batch 1 the block took
// about 1.2 us of a workgroup's 10.  kAhead: rows in flight (the fused
// kernels, which hold their whole state tile here, take 1: more spilled).
template <int LDA, int kAhead>
__device__ __forceinline__ void solve_block16(float (&x)[16], const float* at, int base) {
  static_assert(LDA % 4 == 0, "16-byte aligned rows");
  f32x4 rows[kAhead][4];
  auto fetch = [&](int m, f32x4 (&r)[4]) {
    const f32x4* row = reinterpret_cast<const f32x4*>(at + (base + m) * LDA + base);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (4 * c + 3 > m) r[c] = row[c];  // the chunks holding columns m + 1 .. 15
  };
#pragma unroll
  for (int m = 0; m < kAhead; ++m) fetch(m, rows[m]);
#pragma unroll
  for (int m = 0; m < 15; ++m) {
    f32x4 (&r)[4] = rows[m % kAhead];
    const float xm = x[m];
#pragma unroll
    for (int i = m + 1; i < 16; ++i) x[i] -= r[i >> 2][i & 3] * xm;
    if (m + kAhead < 15) fetch(m + kAhead, r);
    __builtin_amdgcn_sched_barrier(0);  // (no read is hoisted further ahead)
  }
}

__device__ __forceinline__ void materialize16(const float (&x)[16]) {
  asm volatile("" ::"v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]));
  asm volatile("" ::"v"(x[8]), "v"(x[9]), "v"(x[10]), "v"(x[11]), "v"(x[12]), "v"(x[13]), "v"(x[14]), "v"(x[15]));
}

// lane k of each group of 4 lanes, to all 4 (one quad-permute move)
template <int K>
__device__ __forceinline__ float quad_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), K * 0x55, 0xf, 0xf, false));
}

// The same forward substitution on a whole wave: lane 4j + q holds rows
// 4q .. 4q + 3 of column j.  Step m broadcasts x_m (held by lane
// 4j + m / 4) to its column's 4 lanes with one quad-permute move, and each
// lane updates its 4 rows with A's column m there (rows 4q .. 4q + 3 of at's
// row m: one aligned 16-byte read, issued kAhead steps before its use).
// A's entries at and above the diagonal are zero (the tile is masked to
// strict ancestors, which precede a node), so rows i <= m are left as they
// are and each element sees the same fused multiply-adds in the same order
// as in solve_block16: the result is bit-identical.  A step is one move and
// four multiply-adds on the chain instead of up to 15, and one 16-byte read.
// Writes X_bb to x (pitch LDA) at (base, base).
template <int LDA, int kAhead>
__device__ __forceinline__ void solve_block16_wave(const float* at, float* x, int base, int lane) {
  static_assert(LDA % 4 == 0, "16-byte aligned rows");
  const int j = lane >> 2, q = lane & 3;
  f32x4 xv;
#pragma unroll
  for (int r = 0; r < 4; ++r) xv[r] = (4 * q + r == j) ? 1.f : 0.f;
  const float* col = at + base * LDA + base + 4 * q;  // row m of at: col + m LDA
  f32x4 rows[kAhead];
#pragma unroll
  for (int m = 0; m < kAhead; ++m) rows[m] = *reinterpret_cast<const f32x4*>(col + m * LDA);
#pragma unroll
  for (int m = 0; m < 15; ++m) {
    const f32x4 a = rows[m % kAhead];
    if (m + kAhead < 15) rows[m % kAhead] = *reinterpret_cast<const f32x4*>(col + (m + kAhead) * LDA);
    float xm;
    switch (m >> 2) {
      case 0: xm = quad_bcast<0>(xv[m & 3]); break;
      case 1: xm = quad_bcast<1>(xv[m & 3]); break;
      case 2: xm = quad_bcast<2>(xv[m & 3]); break;
      default: xm = quad_bcast<3>(xv[m & 3]); break;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) xv[r] -= a[r] * xm;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) x[(base + 4 * q + r) * LDA + base + j] = xv[r];
}

// acc += A_blk(bi, bm) * B_blk(bm, bj) over one 16x16x16 block product with
// fp32 MFMA; A from a row-major or (transposed) column-major LDS matrix, B
// row-major.  Lane (n, g), k-step s covers k = 4s + g.
template <int LDA, bool A_TRANSPOSED>
__device__ __forceinline__ f32x4 block_mma(f32x4 acc, const float* a, int bi, int bm, const float* bmat, int bj,
                                           int n16, int g4) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int kk = 16 * bm + 4 * s + g4;
    const float av = A_TRANSPOSED ? a[kk * LDA + 16 * bi + n16] : a[(16 * bi + n16) * LDA + kk];
    const float bv = bmat[kk * LDA + 16 * bj + n16];
    acc = mfma_f32_16x16x4(av, bv, acc);
  }
  return acc;
}

// X_ij = -D_i T for T in the accumulator layout (lane (n, g) holds rows
// 4g + r): k-step s takes row 4g + s of T from register s, so T never leaves
// registers; D_i = X_ii is read from LDS with the same permutation.
template <int LDA>
__device__ __forceinline__ f32x4 neg_diag_times(const float* x, int bi, f32x4 T, int n16, int g4) {
  f32x4 acc = {};
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma_f32_16x16x4(x[(16 * bi + n16) * LDA + 16 * bi + 4 * g4 + s], T[s], acc);
  return -acc;
}

template <int LDA>
__device__ __forceinline__ void store_block(float* m, int bi, int bj, f32x4 acc, int n16, int g4) {
#pragma unroll
  for (int r = 0; r < 4; ++r) m[(16 * bi + 4 * g4 + r) * LDA + 16 * bj + n16] = acc[r];
}

// ---------------------------------------------------------------------------
// fused commit of the previous step's accepted path (dft_tree_commit_verify)
// ---------------------------------------------------------------------------
// The previous step's accepted path of one request.  Lane l holds path entry
// l % 16 (loaded before anything else, as a 32-bit word: the low half of an
// int64 entry), so slot lookups are lane shuffles, not indexed arrays.
// Entries c < len with 0 <= e < bound are valid; u is the last valid one.
struct Pending {
  int ent;         // this lane's entry (an invalid one replaced by u)
  uint32_t vmask;  // bit c: entry c valid
  int last;        // slot of u, -1 when nothing is pending
  bool bad;        // an entry within the length names a node past the previous tree
  int64_t prow0;   // row of the request's node 0 in the previous step's buffers
};

// LDS of the recomputed path values: four 16 x 16 matrices (row pitch 17),
// then the 16 key norms of the raw-key form
constexpr int kRvxNorms = 4 * 16 * 17, kRvx = kRvxNorms + 16;

// The recompute's slot of path position i, and the position of slot i (the
// map is its own inverse): positions 4m .. 4m + 3 take slots m, 4 + m, 8 + m,
// 12 + m, the k indices of k-step m of an MFMA 16x16x4 whose B operand is in
// the accumulator layout (k = 4g + m in lane group g).
__device__ __forceinline__ int rvn_slot(int i) { return 4 * (i & 3) + (i >> 2); }

// The 32-bit word of path entry l % 16 (the low half of an int64 entry).
__device__ __forceinline__ const uint32_t* path_word(const dft_pending_commit& c, int b, int lane) {
  const int col = (lane & 15) < c.path_cols ? (lane & 15) : c.path_cols - 1;
  const int esz = c.path_dtype == DFT_I64 ? 8 : 4;
  return reinterpret_cast<const uint32_t*>(static_cast<const char*>(c.path) +
                                           ((int64_t)b * c.path_req_stride + col) * esz);
}

// The request's previous rows and how many path entries count; read with
// the block's other index loads, before any stream is issued.
struct PendingHead {
  int64_t prow0;
  int bound, len;
};

// (CP: a pointer to the descriptor, generic or in the kernel-argument segment)
template <class CP>
__device__ __forceinline__ PendingHead pending_head(CP c, int b) {
  PendingHead ph;
  const int32_t* pcu = c->prev_cu_seqlens;
  if (pcu) {
    ph.prow0 = pcu[b];
    ph.bound = pcu[b + 1] - pcu[b];
  } else {
    ph.prow0 = (int64_t)b * c->prev_n_nodes;
    ph.bound = c->prev_n_nodes;
  }
  ph.len = c->path_cols;
  if (c->path_len) {
    const int64_t l = ld_i(c->path_len, b, c->path_len_dtype);
    ph.len = l < 0 ? 0 : (l < ph.len ? (int)l : ph.len);
  }
  // uniform (one request): kept in scalar registers through phase 1
  ph.prow0 = uniform64(ph.prow0);
  ph.bound = __builtin_amdgcn_readfirstlane(ph.bound);
  ph.len = __builtin_amdgcn_readfirstlane(ph.len);
  return ph;
}

__device__ __forceinline__ Pending decode_pending(const PendingHead& ph, int lane, uint32_t word) {
  Pending pd;
  pd.prow0 = ph.prow0;
  const int bound = ph.bound, len = ph.len;
  const int e = (int)word;
  const bool ok = (lane & 15) < len && e >= 0 && e < bound;
  pd.bad = (__ballot((lane & 15) < len && e >= bound) & 0xffffull) != 0;
  pd.vmask = (uint32_t)__ballot(ok) & 0xffffu;
  pd.last = pd.vmask ? 31 - __clz(pd.vmask) : -1;
  const int u = __shfl(e, pd.last < 0 ? 0 : pd.last);
  pd.ent = ok ? e : (pd.last < 0 ? 0 : u);
  return pd;
}

// The ancestry rows of the pending entries for the walk check
// (c.prev_anc_bits): wave 0's lanes 16-31 copy the low words and lanes 32-47
// the high words of the row of entry lane % 16 into walk[16 .. 47] (row 4
// of the gate words, whose lanes 16-47 nothing else reads).  With nothing
// pending the source is `dummy` (valid memory, never checked).  UNTRACKED:
// the copy is hidden from the backend's wait analysis (issued late, it
// would make every LDS read after it wait for the whole state tile); the
// caller's later loads, which return in order behind it, cover it.
template <bool UNTRACKED>
__device__ __forceinline__ void issue_walk_dma(const dft_pending_commit& c, const Pending& pd, int wave, int lane,
                                               const void* dummy, uint32_t* walk) {
  if (!c.prev_anc_bits || wave != 0 || lane < 16 || lane >= 48) return;
  const uint32_t* src = pd.last >= 0 ? reinterpret_cast<const uint32_t*>(c.prev_anc_bits + pd.prow0 + pd.ent) + (lane >> 5)
                                     : static_cast<const uint32_t*>(dummy);
  if constexpr (UNTRACKED) lds_dma4_untracked(src, walk);
  else lds_dma4(src, walk);
}

// Whether the valid pending entries, in path order, walk down from the
// previous tree's root (uniform): lane c < 16 checks that its entry's
// ancestors-or-self in that tree are exactly the valid entries 0 .. c and
// that none of them repeats, which makes entry c the child of the valid
// entry before it.  The recomputed values and the closed-form commit both
// assume this (fc1_fused.py:41 checks path ancestry on the device).
__device__ __forceinline__ bool pending_walk_ok(const Pending& pd, int lane, const uint32_t* walk, int bound) {
  const int c = lane & 15, e = pd.ent;
  const bool valid = (pd.vmask >> c) & 1u;
  uint64_t m = (valid && e < 64) ? (1ull << e) : 0ull;  // entries past 63 cannot be rows of a tree here
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {  // inclusive OR over positions 0 .. c
    const uint32_t lo = __shfl_up((uint32_t)m, o, 16), hi = __shfl_up((uint32_t)(m >> 32), o, 16);
    if (c >= o) m |= ((uint64_t)hi << 32) | lo;
  }
  const uint64_t anc = (((uint64_t)walk[32 + c] << 32) | walk[16 + c]) & mask_upto(e) & mask_below(bound);
  const int cnt = __popc(pd.vmask & ((2u << c) - 1u));
  const bool ok = !valid || (e < 64 && __popcll(m) == cnt && anc == m);
  return (__ballot(!ok) & 0xffffull) == 0;
}

// Two 16-byte pieces of the path keys per thread (path slot 4w + g, columns
// 4n .. and 64 + 4n ..), each lane's B-operand values vn_p[v] and gains G_p
// for path slots p = 4s + g.  With nothing pending the sources are the state
// tile itself (valid memory, never used): the loads are issued on every path,
// so that no register is left waiting on a load that only some paths issue
// (the compiler would then make later code wait for every store since).

// (NW = 8: one 16-byte piece per thread, columns 4n + 64 (w / 4) ..)
//
// RAWK: the keys are the previous step's raw bf16 rows (c.key_rows), read as
// two 8-byte pieces per thread (columns 4n .. and 64 + 4n .., both at NW = 8
// too: the 16 lanes of a slot then hold its whole row, for the norm) and
// normalised when they are staged.
template <int NW, bool RAWK>
struct PathKeys {
  f32x4 k[8 / NW];
};
template <int NW>
struct PathKeys<NW, true> {
  uint2 raw[2];
};
// The path's values and gains as a thread holds them until the commit: the
// saved vn_p[v] and G_p of slots p = 4s + g, or (RVN: recomputed values) the
// previous step's raw bf16 value rows of path positions 4e + g (slots 4g + e
// of the recompute, the rows of W's accumulator layout; vr[e][t]: tile t's
// column, two bf16 per register), with the gain and b gate of position
// lane % 16.
template <int NW, bool RVN>
struct PathVals {
  float v[4][Waves<NW>::TT];
  float g[4];
};
template <int NW>
struct PathVals<NW, true> {
  u16x2 vr[4];
  float gl, bl;
};
template <int NW, bool RAWK, bool RVN>
__device__ __forceinline__ void issue_pending(const dft_pending_commit& c, const Pending& pd, int h, int wave, int lane,
                                              const float* dummy, PathKeys<NW, RAWK>& pk, PathVals<NW, RVN>& pv) {
  constexpr int KP = 8 / NW, TT = Waves<NW>::TT, CW = Waves<NW>::CW;
  const bool any = pd.last >= 0;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int krow = __shfl(pd.ent, 4 * (wave & 3) + g4);
  if constexpr (RAWK) {
    const uint16_t* kb = any ? c.key_rows + (int64_t)(h / c.k_head_div) * c.kr_h_stride + pd.prow0 * c.kr_row_stride
                             : reinterpret_cast<const uint16_t*>(dummy);
    const int64_t ks = any ? c.kr_row_stride : 0;
#pragma unroll
    for (int m = 0; m < 2; ++m) pk.raw[m] = *reinterpret_cast<const uint2*>(kb + krow * ks + 4 * n16 + 64 * m);
  } else {
    const float* kb = any ? c.keys + (int64_t)(h / c.k_head_div) * c.k_h_stride + pd.prow0 * c.k_row_stride : dummy;
    const int64_t ks = any ? c.k_row_stride : 0;
#pragma unroll
    for (int m = 0; m < KP; ++m)
      pk.k[m] = *reinterpret_cast<const f32x4*>(kb + krow * ks + 4 * (n16 + 16 * (m + KP * (wave >> 2))));
  }
  const float* gb = any ? c.gains + (int64_t)h * c.g_h_stride + pd.prow0 * c.g_row_stride : dummy;
  const int64_t gs = any ? c.g_row_stride : 0;
  if constexpr (RVN) {
    const uint16_t* vb = any ? c.value_rows + (int64_t)h * c.vr_h_stride + pd.prow0 * c.vr_row_stride
                             : reinterpret_cast<const uint16_t*>(dummy);
    const int64_t vs = any ? c.vr_row_stride : 0;
    static_assert(TT <= 2, "two bf16 per register");
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t row = __shfl(pd.ent, 4 * e + g4);  // slot 4g + e is position 4e + g
#pragma unroll
      for (int t = 0; t < TT; ++t) pv.vr[e][t] = vb[row * vs + CW * wave + 16 * t + n16];
    }
    pv.gl = gb[pd.ent * gs];
    // the b gate as the verify reads it: the whole 32-bit word, converted later
    uint32_t sh;
    const uint32_t* bw = any ? word_of(c.prev_b, (pd.prow0 + pd.ent) * c.pb_row_stride + h, c.prev_b_dtype, sh)
                             : reinterpret_cast<const uint32_t*>(dummy);
    pv.bl = word_to_f(*bw, any ? sh : 0u, any ? c.prev_b_dtype : (int)DFT_F32);
  } else {
    const float* vb = any ? c.values + (int64_t)h * c.v_h_stride + pd.prow0 * c.v_row_stride : dummy;
    const int64_t vs = any ? c.v_row_stride : 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int row = __shfl(pd.ent, 4 * s + g4);
#pragma unroll
      for (int t = 0; t < TT; ++t) pv.v[s][t] = vb[row * vs + CW * wave + 16 * t + n16];
      pv.g[s] = gb[row * gs];
    }
  }
}

// (32-wide recompute form with raw key rows) The path's raw k and v rows
// copied into LDS ahead of the state tile, so that they do not queue behind
// it: key slot s (position rvn_slot(s)) at row s of praw, value position p
// at row 16 + p, both in the q/k row layout; the gains (lanes 0-15) and the
// b-gate words (lanes 16-31) at rvx[0 .. 31], which the recompute claims only
// after path_from_lds has read them.
template <int NW>
__device__ __forceinline__ void issue_path_dma(const dft_pending_commit& c, const Pending& pd, int h, int wave,
                                               int lane, const float* dummy, uint16_t* praw, float* rvx) {
  static_assert(NW == 4, "one key and one value copy per wave");
  const bool any = pd.last >= 0;
  const int cp = lane & 15, s = 4 * wave + (lane >> 4);
  const int krow = __shfl(pd.ent, rvn_slot(s));
  const int vrow = __shfl(pd.ent, s);
  const uint16_t* kb = any ? c.key_rows + (int64_t)(h / c.k_head_div) * c.kr_h_stride + pd.prow0 * c.kr_row_stride
                           : reinterpret_cast<const uint16_t*>(dummy);
  const uint16_t* vb = any ? c.value_rows + (int64_t)h * c.vr_h_stride + pd.prow0 * c.vr_row_stride
                           : reinterpret_cast<const uint16_t*>(dummy);
  const int64_t ks = any ? c.kr_row_stride : 0, vs = any ? c.vr_row_stride : 0;
  const int ck = 8 * ((cp ^ s) & 15);  // the chunk that lands at chunk position cp of row s
  lds_dma16(kb + krow * ks + ck, praw + 4 * wave * kD);
  lds_dma16(vb + vrow * vs + ck, praw + (16 + 4 * wave) * kD);
  if (wave == 0 && lane < 32) {
    const void* src;
    if (lane < 16) {
      src = any ? static_cast<const void*>(c.gains + (int64_t)h * c.g_h_stride + (pd.prow0 + pd.ent) * c.g_row_stride)
                : static_cast<const void*>(dummy);
    } else {
      uint32_t sh;
      src = any ? static_cast<const void*>(word_of(c.prev_b, (pd.prow0 + pd.ent) * c.pb_row_stride + h,
                                                   c.prev_b_dtype, sh))
                : static_cast<const void*>(dummy);
    }
    lds_dma4(src, rvx);
  }
}
// The keys, gains and b gates issue_pending would have loaded, read from
// those copies (the values are read where W is formed: path_values<VLDS>).
template <int NW>
__device__ __forceinline__ void path_from_lds(const dft_pending_commit& c, const Pending& pd, int h, int wave,
                                              int lane, const uint16_t* praw, const float* rvx,
                                              PathKeys<NW, true>& pk, PathVals<NW, true>& pv) {
  const int n16 = lane & 15, g4 = lane >> 4;
  const int rs = rvn_slot(4 * (wave & 3) + g4);
#pragma unroll
  for (int m = 0; m < 2; ++m) pk.raw[m] = *reinterpret_cast<const uint2*>(&praw[qkv_at(rs, 4 * n16 + 64 * m)]);
  pv.gl = rvx[n16];
  const bool any = pd.last >= 0;
  uint32_t sh = 0;
  if (any) (void)word_of(c.prev_b, (pd.prow0 + pd.ent) * c.pb_row_stride + h, c.prev_b_dtype, sh);
  pv.bl = word_to_f(__float_as_uint(rvx[16 + n16]), any ? sh : 0u, any ? c.prev_b_dtype : (int)DFT_F32);
}

// Whole-line state loads (the 32-wide fused form).  In the MFMA layout
// (s0r[t][j] = S0[k = 16j + 4g + e][v = CW w + 16t + n]) one load covers 64
// bytes of each of 16 rows, and a line's two halves come from two
// instructions; a memory-only probe of this tile shape read 128 MiB in
// 24.5 us that way and in 20.9 us as whole lines.  So load (t, 2s + e) reads
// rows 8e + r of tile t (r = lane & 7), chunk 8s + 4 b3 + g of each (b3 =
// lane bit 3, g = lane >> 4): 8 whole lines per instruction, each line over
// 8 lanes 8 apart.  lines_to_mfma then swaps lane bit 3 with e, giving rows
// 8 b3 + r = n at chunks 8s + g (j = 2s) and 8s + 4 + g (j = 2s + 1).
// Fused kernel at batch 64: 73.2 -> 71.8 us.  The verify kernels keep the
// MFMA layout: the 32-wide one gained nothing (its state groups stream in
// under phase 1), and the 64-wide ones, latency-bound, lost 3% to the swap.
__device__ __forceinline__ float row_ror8(float x) {  // lane l ^ 8 of the same 16-lane row
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}
__device__ __forceinline__ void lines_to_mfma(f32x4& a, f32x4& b, bool b3) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // one lane move per pair: u's row_ror8 is b of lane l ^ 8 where b3 is
    // set, a of lane l ^ 8 where it is not
    const float ru = row_ror8(b3 ? a[e] : b[e]);
    a[e] = b3 ? ru : a[e];
    b[e] = b3 ? b[e] : ru;
  }
}
// k-step group s of a tile loaded by issue_state / issue_state_group
template <int NW>
__device__ __forceinline__ void state_group_to_mfma(f32x4 (&s0r)[Waves<NW>::TT][8], int s, int lane) {
  const bool b3 = (lane >> 3) & 1;
#pragma unroll
  for (int t = 0; t < Waves<NW>::TT; ++t) lines_to_mfma(s0r[t][2 * s], s0r[t][2 * s + 1], b3);
}
template <int NW>
__device__ __forceinline__ void state_to_mfma(f32x4 (&s0r)[Waves<NW>::TT][8], int lane) {
#pragma unroll
  for (int s = 0; s < 4; ++s) state_group_to_mfma<NW>(s0r, s, lane);
}

// s0r <- e^{G_u} s0r + sum_p e^{G_u - G_p} k_p vn_p^T on the wave's tiles
// (s0r[t][j] is the accumulator of a 16x16 MFMA with rows k = 16j + 4g + r and
// columns v = 32w + 16t + n): fp32 MFMA 16x16x4, path slots as the inner
// dimension (A = keys from LDS, B = weighted values from registers).
// thread (w, l) holds chunks n and n + 16 of the key of path slot 4w + g
// (NW = 8: chunk n + 16 (w / 4) of path slot 4 (w % 4) + g)
// Raw keys are normalised as the verify normalises its k rows, k / sqrt(sum
// k^2 + 1e-6) (the sum over the slot's 16 lanes, so in another order than
// the verify's: the staged keys can differ from its saves by an ulp).
template <int NW, bool RAWK, bool RVN>
__device__ __forceinline__ void stage_pending_keys(float* pkey, float* rvx, const PathKeys<NW, RAWK>& pk, int wave,
                                                   int lane) {
  constexpr int KP = 8 / NW;
  const int n16 = lane & 15;
  const int rp = 4 * (wave & 3) + (lane >> 4);  // the path position loaded
  const int rs = RVN ? rvn_slot(rp) : rp;      // its staging slot
  if constexpr (RAWK) {
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk.raw[m].x), __builtin_bit_cast(bf16x2, pk.raw[m].x),
                                           ss, false);
      ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk.raw[m].y), __builtin_bit_cast(bf16x2, pk.raw[m].y),
                                           ss, false);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o);
    const float rn = rsqrtf(ss + 1e-6f);
    if constexpr (RVN) {
      // the raw rows in the q/k row layout (bf16 MFMA operands for the
      // recompute) and the norms beside the recompute's matrices
      uint16_t* praw = reinterpret_cast<uint16_t*>(pkey);
#pragma unroll
      for (int m = 0; m < KP; ++m) {
        const int mm = m + KP * (wave >> 2);
        *reinterpret_cast<uint2*>(&praw[qkv_at(rs, 4 * n16 + 64 * mm)]) = mm == 0 ? pk.raw[0] : pk.raw[1];
      }
      if (n16 == 0 && wave < 4) rvx[kRvxNorms + rs] = rn;
      return;
    }
#pragma unroll
    for (int m = 0; m < KP; ++m) {
      const int mm = m + KP * (wave >> 2);  // 0 or 1 (uniform)
      const uint2 u = mm == 0 ? pk.raw[0] : pk.raw[1];
      const f32x4 v = {__uint_as_float(u.x << 16) * rn, __uint_as_float(u.x & 0xffff0000u) * rn,
                       __uint_as_float(u.y << 16) * rn, __uint_as_float(u.y & 0xffff0000u) * rn};
      *reinterpret_cast<f32x4*>(&pkey[pkey_at(rs, 4 * (n16 + 16 * mm))]) = v;
    }
  } else {
#pragma unroll
    for (int m = 0; m < KP; ++m)
      *reinterpret_cast<f32x4*>(&pkey[pkey_at(rs, 4 * (n16 + 16 * (m + KP * (wave >> 2))))]) = pk.k[m];
  }
}

// e^{G_u}, the decay of the whole path, broadcast from the lane that holds G_u
__device__ __forceinline__ float pending_decay_log(const Pending& pd, const float (&gp)[4]) {
  const int cu = pd.last, su = cu >> 2;
  const float gsel = su == 0 ? gp[0] : su == 1 ? gp[1] : su == 2 ? gp[2] : gp[3];
  return __shfl(gsel, (cu & 3) * 16);
}

// hi/lo bf16 splits of columns 32s + 4g .. + 3 and 32s + 16 + 4g .. + 3 of
// staged key p: the A (and B) operand of k-step s of a bf16 MFMA 16x16x32
// whose B operand is k-step group s of the state tile
__device__ __forceinline__ void pkey_split(const float* pkey, int p, int s, int g4, bf16x8& hi, bf16x8& lo) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(&pkey[pkey_at(p, 32 * s + 4 * g4)]);
  const f32x4 b = *reinterpret_cast<const f32x4*>(&pkey[pkey_at(p, 32 * s + 16 + 4 * g4)]);
  const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  split_bf16x8(x, hi, lo);
}

// D = C + P Q for 16 x 16 row-major LDS matrices (row pitch 17), fp32 MFMA
// 16x16x4 (k-step m covers k = 4g + m); C and D in the accumulator layout
// (element e of lane (n, g): row 4g + e, column n).  One wave's LDS
// operations run in order, so a product may read what the wave stored just
// before and store over an operand it has read.
__device__ __forceinline__ f32x4 mat16_mul(const float* P, const float* Q, f32x4 acc, int n16, int g4) {
#pragma unroll
  for (int m = 0; m < 4; ++m) acc = mfma_f32_16x16x4(P[n16 * 17 + 4 * g4 + m], Q[(4 * g4 + m) * 17 + n16], acc);
  return acc;
}
__device__ __forceinline__ void mat16_store(float* D, f32x4 acc, int n16, int g4) {
#pragma unroll
  for (int e = 0; e < 4; ++e) D[(4 * g4 + e) * 17 + n16] = acc[e];
}

// RVN: the values of the path's slots, recomputed from the tile before the
// commit.  For a root walk the ancestors of every path node are the path's
// earlier nodes, so vn_path = X W over the path alone: A_pq = beta_p (k_p .
// k_q) e^{G_p - G_q} for valid q < p, X = (I + A)^-1, and W_p = beta_p (v_p -
// e^{G_p} S0^T k_p) with S0 the tile as the previous verify read it.
//  * wave 0 forms the 16 x 16 Gram of the staged keys by bf16 MFMA 16x16x32
//    (RAWK: on the raw bf16 rows, exact products, then scaled by the two
//    norms; else on hi/lo splits of the fp32 keys, three products), and X =
//    (I + A)^-1 as the product (I - A)(I + A^2)(I + A^4)(I + A^8), exact for
//    A strictly lower triangular in path order: with the path's last valid
//    position at len - 1, A^len = 0, so the factors and powers from A^len on
//    are skipped (fp32 MFMA 16x16x4 products through LDS matrices; a path of
//    up to 4 positions takes two, up to 2 none).  A forward substitution holds a 16-float
//    column per lane, which beside the tile spilled the 32-wide kernel;
//  * Ck = K S0 by bf16 MFMA 16x16x32 on the tile registers split into hi/lo
//    bf16 (as the verify's Cq/Ck pass splits them; RAWK: the raw rows, exact,
//    the norm applied to the result, two products per k-step; else three),
//    rows = slots 4g + e, and W in place, zero on invalid slots (so vn is
//    zero there).  The MFMA work here lies on every workgroup's critical
//    path: at batch 64 the fp32 MFMA 16x16x4 form of Ck cost 4 us per launch,
//    this one about 1;
//  * vn = X W by fp32 MFMA 16x16x4.  The keys are staged at rvn_slot of their
//    path position, so k-step m of this product covers positions 4m .. 4m +
//    3 (a path of up to 4 positions takes one k-step, not four), and element
//    s of a lane (slot 4g + s) is position 4s + g: the B-operand layout of
//    the commit below (vnr[s] = position 4s + g), which reads the key of
//    position p from slot rvn_slot(p).
// Every thread arrives here (one barrier, skipped by the whole workgroup
// when nothing is pending).
// VLDS: the raw value rows are in LDS (rows 16 + position of the key
// staging, issue_path_dma) rather than in pv.vr.
template <int NW, bool RAWK, bool VLDS = false>
__device__ __forceinline__ void path_values(const Pending& pd, const float* pkey, float* rvx,
                                            const PathVals<NW, true>& pv, int wave, int lane,
                                            const f32x4 (&s0r)[Waves<NW>::TT][8], float (&vnr)[4][Waves<NW>::TT]) {
  constexpr int TT = Waves<NW>::TT;
  const int n16 = lane & 15, g4 = lane >> 4;
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int t = 0; t < TT; ++t) vnr[s][t] = 0.f;
  if (pd.last < 0) return;  // uniform
  const u16x2 (&vr)[4] = pv.vr;
  const float beta = 1.f / (1.f + expf(-pv.bl));  // slot lane % 16, as the verify forms beta
  if (wave == 0) {
    // (lane ids laundered in each part: addresses computed where used)
    int lg = lane;
    asm volatile("" : "+v"(lg));
    const int n16 = lg & 15, g4 = lg >> 4;
    // the Gram K K^T by bf16 MFMA 16x16x32 (the A and B operands are the same
    // values): k-step s covers columns 32s + 4g .. + 3 and 32s + 16 + 4g .. + 3
    // of slot n
    f32x4 gk = {};
    if constexpr (RAWK) {  // the raw rows: exact products, normed below
      const uint16_t* praw = reinterpret_cast<const uint16_t*>(pkey);
      const int op = qkv_op4(n16, g4);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 kr = lds_bf16x8_split(praw + (op ^ (32 * s)), praw + (op ^ (32 * s + 16)));
        gk = mfma_bf16_16x16x32(kr, kr, gk);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        bf16x8 kh, kl;
        pkey_split(pkey, n16, s, g4, kh, kl);
        gk = mfma_bf16_16x16x32(kh, kh, gk);
        gk = mfma_bf16_16x16x32(kh, kl, gk);
        gk = mfma_bf16_16x16x32(kl, kh, gk);
      }
    }
    // slots p = 4g + e (row) and n (column), at path positions rvn_slot(p)
    // and rvn_slot(n): A_pn is on where n's position precedes p's
    const int iq = rvn_slot(n16);
    const float gq = __shfl(pv.gl, iq), rq = RAWK ? rvx[kRvxNorms + n16] : 1.f;
    const bool okq = (pd.vmask >> iq) & 1u;
    f32x4 ia;  // I - A in the accumulator layout
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int p = 4 * g4 + e, ip = 4 * e + g4;  // element e of lane (n, g): A[4g + e][n]
      const bool on = iq < ip && okq && ((pd.vmask >> ip) & 1u);
      // (the shuffles outside the select: inside it they become a branch,
      // and a lane reads another that the branch has switched off)
      const float bp = __shfl(beta, ip), gpp = __shfl(pv.gl, ip);
      const float rp = RAWK ? rvx[kRvxNorms + p] : 1.f;
      const float a = on ? bp * __expf(gpp - gq) * (rp * rq * gk[e]) : 0.f;
      rvx[p * 17 + n16] = a;
      ia[e] = (p == n16 ? 1.f : 0.f) - a;
    }
    float* a2 = rvx + 16 * 17;
    float* a4 = rvx + 2 * 16 * 17;
    float* a8 = rvx + 3 * 16 * 17;
    const f32x4 zero = {};
    const int len = pd.last + 1;  // A^len = 0 (uniform)
    f32x4 x = ia;                 // I - A: X when A^2 = 0
    if (len > 2) {
      mat16_store(a2, mat16_mul(rvx, rvx, zero, n16, g4), n16, g4);
      if (len > 4) mat16_store(a4, mat16_mul(a2, a2, zero, n16, g4), n16, g4);
      if (len > 8) mat16_store(a8, mat16_mul(a4, a4, zero, n16, g4), n16, g4);
#pragma unroll
      for (int m = 0; m < 4; ++m) {  // (I - A) + (I - A) A^2
        const int k = 4 * g4 + m;
        x = mfma_f32_16x16x4((n16 == k ? 1.f : 0.f) - rvx[n16 * 17 + k], a2[k * 17 + n16], x);
      }
      if (len > 4) {
        mat16_store(a2, x, n16, g4);
        x = mat16_mul(a2, a4, x, n16, g4);  // ... (I + A^4)
      }
      if (len > 8) {
        mat16_store(a2, x, n16, g4);
        x = mat16_mul(a2, a8, x, n16, g4);  // ... (I + A^8)
      }
    }
    mat16_store(rvx, x, n16, g4);  // X over A
  }
  // Ck by bf16 MFMA 16x16x32 on the tile registers: k-step s takes groups 2s
  // and 2s + 1 of the tile, k = 32s + 4g + e and 32s + 16 + 4g + e, as the
  // key operand does.  (Its key reads stay below the solve: hoisted above it,
  // they and the solve's operands together spilled at the 32-wide kernel's
  // register cap.)
  asm volatile("" ::: "memory");
  int lk = lane;
  asm volatile("" : "+v"(lk));
  const int n16k = lk & 15, g4k = lk >> 4;
  f32x4 w[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) w[t] = f32x4{};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8 kh, kl;
    if constexpr (RAWK) {
      const uint16_t* praw = reinterpret_cast<const uint16_t*>(pkey);
      const int op = qkv_op4(n16k, g4k);
      kh = lds_bf16x8_split(praw + (op ^ (32 * s)), praw + (op ^ (32 * s + 16)));
    } else {
      pkey_split(pkey, n16k, s, g4k, kh, kl);
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const float xs[8] = {s0r[t][2 * s][0],     s0r[t][2 * s][1],     s0r[t][2 * s][2],     s0r[t][2 * s][3],
                           s0r[t][2 * s + 1][0], s0r[t][2 * s + 1][1], s0r[t][2 * s + 1][2], s0r[t][2 * s + 1][3]};
      bf16x8 sh, sl;
      split_bf16x8(xs, sh, sl);
      w[t] = mfma_bf16_16x16x32(kh, sh, w[t]);
      w[t] = mfma_bf16_16x16x32(kh, sl, w[t]);
      if constexpr (!RAWK) w[t] = mfma_bf16_16x16x32(kl, sh, w[t]);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int p = 4 * g4 + e, ip = 4 * e + g4;  // slot, position
    const float bp = __shfl(beta, ip);
    const float ep = __expf(__shfl(pv.gl, ip)) * (RAWK ? rvx[kRvxNorms + p] : 1.f);
    const bool ok = (pd.vmask >> ip) & 1u;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const uint16_t vb = VLDS ? reinterpret_cast<const uint16_t*>(pkey)[qkv_at(16 + ip, Waves<NW>::CW * wave + 16 * t + n16)]
                               : vr[e][t];
      w[t][e] = ok ? bp * (bf16_bits_to_f32(vb) - ep * w[t][e]) : 0.f;
    }
  }
  __syncthreads();  // X complete
  f32x4 vn[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) vn[t] = f32x4{};
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (4 * m > pd.last) break;  // uniform: k-step m holds positions 4m .. 4m + 3
    const float a = rvx[n16 * 17 + 4 * g4 + m];  // X[n][k = 4g + m]; B = W[4g + m][v], element m
#pragma unroll
    for (int t = 0; t < TT; ++t) vn[t] = mfma_f32_16x16x4(a, w[t][m], vn[t]);
  }
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int t = 0; t < TT; ++t) vnr[s][t] = vn[t][s];
}

// The commit of a landed tile (a no-op when nothing is pending; the tile
// leaves in the MFMA layout either way).  pkey: 16 x 128 floats of LDS that
// no other wave touches until the next barrier; every thread arrives here
// (the staging is followed by a barrier).  LINES: the tile was loaded as
// whole lines, and is turned into the MFMA layout after the keys are staged:
// they were loaded after it, so it has landed, and their registers are free
// by then.  walk: the entries' ancestry rows (issue_walk_dma, landed before
// the keys the staging waits for), or null for no walk check; a path that
// fails it is dropped here (pd then says nothing is pending, and the caller
// writes nothing back).
template <int NW, bool LINES, bool RAWK, bool RVN, bool VLDS = false>
__device__ __forceinline__ void commit_tile(Pending& pd, float* pkey, float* rvx, const PathKeys<NW, RAWK>& kr,
                                            const PathVals<NW, RVN>& pv, int wave, int lane,
                                            f32x4 (&s0r)[Waves<NW>::TT][8], const uint32_t* walk, int bound) {
  constexpr int TT = Waves<NW>::TT;
  const int n16 = lane & 15, g4 = lane >> 4;
  stage_pending_keys<NW, RAWK, RVN>(pkey, rvx, kr, wave, lane);
  __syncthreads();
  if (walk && !pending_walk_ok(pd, lane, walk, bound)) {  // uniform
    pd.last = -1;
    pd.vmask = 0;
  }
  if constexpr (LINES) state_to_mfma<NW>(s0r, lane);
  float gp[4], vnr[4][TT];
  if constexpr (RVN) {
    // The swapped tile in registers of its own: left to itself the compiler
    // sinks the swap's selects into their first use, the recompute's MFMAs,
    // and holds the unswapped tile and the rotated halves (96 registers)
    // until then.  (No instruction crosses the scheduling barriers: the value
    // loads and gain shuffles hoisted into the swap were spilled.)
    if constexpr (LINES)
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("" : "+v"(s0r[t][j]));
    __builtin_amdgcn_sched_barrier(0);
    path_values<NW, RAWK, VLDS>(pd, pkey, rvx, pv, wave, lane, s0r, vnr);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 4; ++s) gp[s] = __shfl(pv.gl, 4 * s + g4);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      gp[s] = pv.g[s];
#pragma unroll
      for (int t = 0; t < TT; ++t) vnr[s][t] = pv.v[s][t];
    }
  }
  const float gu = pending_decay_log(pd, gp);
  const float eu = pd.last >= 0 ? __expf(gu) : 1.f;
  // RVN: the loop's key addresses from an opaque lane id, so that they are
  // computed here rather than held (and spilled) through the recompute
  int lane_c = lane;
  if constexpr (RVN) asm volatile("" : "+v"(lane_c));
  const int n16c = lane_c & 15, g4c = lane_c >> 4;
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) s0r[t][j] *= eu;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (4 * s > pd.last) break;  // uniform
    const int p = 4 * s + g4c;
    const float wgt = ((pd.vmask >> p) & 1u) ? __expf(gu - gp[s]) : 0.f;
    float bv[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) bv[t] = wgt * vnr[s][t];
    // (raw-key recompute form: the raw rows staged, normed as they are read,
    // which rounds as the staged fp32 keys of the other forms do)
    const int ks = RVN ? rvn_slot(p) : p;  // the key's staging slot
    const float rkp = (RAWK && RVN) ? rvx[kRvxNorms + ks] : 1.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float av = (RAWK && RVN) ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(pkey)[qkv_at(ks, 16 * j + n16c)]) * rkp
                                     : pkey[pkey_at(ks, 16 * j + n16c)];
#pragma unroll
      for (int t = 0; t < TT; ++t) s0r[t][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv[t], s0r[t][j], 0, 0, 0);
    }
  }
}

// k-step group s of the state tile (j = 2s, 2s + 1 of every column tile).
// LINES: as whole lines (state_group_to_mfma turns it into the MFMA layout);
// otherwise straight into the MFMA layout.
template <bool NT, bool LINES, int NW>
__device__ __forceinline__ void issue_state_group(const float* S0, int64_t v_stride, int wave, int lane, int s,
                                                  f32x4 (&s0r)[Waves<NW>::TT][8]) {
  const int n16 = lane & 15, g4 = lane >> 4;
  const int r8 = lane & 7, c8 = 4 * ((lane >> 3) & 1) + g4;  // LINES: row in 8, chunk in the line
#pragma unroll
  for (int t = 0; t < Waves<NW>::TT; ++t) {
    const float* rowp = LINES ? S0 + (int64_t)(Waves<NW>::CW * wave + 16 * t + r8) * v_stride + 4 * c8 + 32 * s
                              : S0 + (int64_t)(Waves<NW>::CW * wave + 16 * t + n16) * v_stride + 4 * g4 + 32 * s;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const f32x4* src = reinterpret_cast<const f32x4*>(LINES ? rowp + (int64_t)(8 * e) * v_stride : rowp + 16 * e);
      s0r[t][2 * s + e] = NT ? __builtin_nontemporal_load(src) : *src;
    }
  }
}

// The committed tile goes back where it was read, as whole 128-byte lines.
// In the MFMA layout a lane group holds 64 bytes of each of 16 rows, so a
// direct store writes half lines; non-temporal half lines reach memory
// unmerged, and ordinary stores are slower still (fused kernel at batch 64:
// 81.2 us with half-line non-temporal stores, 84.8 with ordinary ones).  So
// each 16-row x 32-column piece (registers j = 2s, 2s + 1 of tile t) goes
// through the wave's own 2 KiB of LDS, `stage`, and comes back as 8 lanes
// per 128-byte row.  The piece's rows are 32 floats, so 16-byte chunk c of
// row r sits at chunk c ^ (r & 7): the writes (8 lanes = 8 rows at one
// chunk) and the read-backs (8 lanes = 8 chunks of one row) then hit 32
// distinct banks.  A wave's LDS operations run in order, so the buffer is
// reused piece after piece without waits.
template <int NW>
__device__ __forceinline__ void store_state(float* S, int64_t v_stride, int wave, int lane,
                                            const f32x4 (&s0r)[Waves<NW>::TT][8], float* stage) {
  const int n16 = lane & 15, g4 = lane >> 4;
  const int r8 = lane >> 3, c8 = lane & 7;
  const int64_t step8 = 8 * v_stride;
  f32x4* st = reinterpret_cast<f32x4*>(stage);  // 8 chunks of 16 bytes per row
  f32x4* w0 = st + 8 * n16 + (g4 ^ (n16 & 7));
  f32x4* w1 = st + 8 * n16 + ((4 + g4) ^ (n16 & 7));
  const f32x4* rd = st + 8 * r8 + (c8 ^ r8);  // rows r8 and 8 + r8 share the swizzle
#pragma unroll
  for (int t = 0; t < Waves<NW>::TT; ++t) {
    float* r0 = S + (int64_t)(Waves<NW>::CW * wave + 16 * t + r8) * v_stride + 4 * c8;  // rows r8, 8 + r8 of the tile
    float* r1 = r0 + step8;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // row n16 of the piece (tile t, columns 32 s ..): columns 4 g4 .. and 16 + 4 g4 ..
      *w0 = s0r[t][2 * s];
      *w1 = s0r[t][2 * s + 1];
      const f32x4 v0 = rd[0], v1 = rd[64];
      __builtin_nontemporal_store(v0, reinterpret_cast<f32x4*>(r0 + 32 * s));
      __builtin_nontemporal_store(v1, reinterpret_cast<f32x4*>(r1 + 32 * s));
    }
  }
}

// ---------------------------------------------------------------------------
// the verify, phase by phase.  RW holds the q/k/v rows (q, k, v), WK the
// per-head O(N^2) work arrays (am, x, gc, G, beta, rq, rk, cO, anc); the
// caller places the barriers between phases.
// ---------------------------------------------------------------------------
// One (request, v-head) of a launch.
struct Item {
  int b, hk, rr, h;  // request, k-head, v-head within the k-head, v-head
  int n;             // nodes (0: nothing to verify)
  bool span_bad;     // row span negative or past n_nodes (cut to n_nodes): DFT_STATUS_SPAN
  bool no_slot = false;  // negative state index: S0 is read from slot 0, nothing is committed
  int64_t row0;      // row of node 0
  const float* S0;   // the head's state tile (k stride 1 on the vector paths)
};

// block id -> (request, v-head); the R v-heads sharing a k-head get ids 8
// apart so that they land on the same XCD (shared q/k rows in its L2)
// over `batch` requests (a bijection of [0, batch * hv))
__device__ __forceinline__ void item_heads(const dft_verify_args& p, int batch, int id, Item& it) {
  const int R = p.hv / p.hk;
  const int pairs = batch * p.hk;
  const int full = (pairs / 8) * 8 * R;
  int pair, rr;
  if (id < full) {
    const int grp = id / (8 * R), rem = id - grp * 8 * R;
    rr = rem >> 3;
    pair = grp * 8 + (rem & 7);
  } else {
    const int t = id - full;
    pair = (pairs / 8) * 8 + t / R;
    rr = t % R;
  }
  it.b = pair / p.hk;
  it.hk = pair - it.b * p.hk;
  it.rr = rr;
  it.h = it.hk * R + rr;
}
__device__ __forceinline__ void item_heads(const dft_verify_args& p, int id, Item& it) {
  item_heads(p, p.batch, id, it);
}

// rows, node count and state tile of a request (loads the index arrays).
// A row span that is negative or exceeds n_nodes is cut to [0, n_nodes] and
// flagged.  Returns false when the request belongs to the other kernel of a
// launch split by tree size (its node count outside [n_lo, n_hi]).
//
// With size-order records (cls >= 0) the block's request index q counts the
// kernel's own class: record q from the front (class 0) or from the back
// (class 1), read with the class counts in one pair of independent loads;
// q past the class's count exits (those blocks come last in the grid).
// Records whose header names another n_nodes or batch than the launch's are
// ignored (block q then takes request q, as without records).
template <int NP>
__device__ __forceinline__ bool item_rows(const dft_verify_args& p, Item& it, int n_lo, int n_hi, int cls) {
  int span;
  bool rec = false;
  if (cls >= 0) {
    const int4* ord = reinterpret_cast<const int4*>(p.size_order);
    const int q = it.b;
    const int4 hd = ord[0];
    const int4 e = ord[1 + (cls == 0 ? q : p.batch - 1 - q)];
    rec = hd.z == p.n_nodes && hd.w == p.batch;  // uniform
    if (rec) {
      if (q >= (cls == 0 ? hd.x : hd.y)) return false;
      it.b = e.x;
      it.row0 = e.y;
      span = e.z;
    }
  }
  if (!rec) {
    if (p.cu_seqlens) {
      it.row0 = p.cu_seqlens[it.b];
      span = p.cu_seqlens[it.b + 1] - p.cu_seqlens[it.b];
    } else {
      it.row0 = (int64_t)it.b * p.n_nodes;
      span = p.n_nodes;
    }
  }
  it.span_bad = span < 0 || span > p.n_nodes;
  it.n = span < 0 ? 0 : (span > p.n_nodes ? p.n_nodes : span);
  if (it.n < n_lo || it.n > n_hi) return false;
  it.n = it.n > NP ? NP : it.n;  // the launch width covers n_nodes: never cuts
  int64_t slot = it.b;
  if (p.state_indices) {
    slot = ld_i(p.state_indices, it.b, p.state_indices_dtype);
    it.no_slot = slot < 0;
    if (slot < 0) slot = 0;
  }
  it.S0 = p.state + slot * p.state_slot_stride + (int64_t)it.h * p.state_h_stride;
  return true;
}

// Wave 0's lane i fetches node i's gate words and ancestry bits into graw
// (rows past the tree repeat the last node; the request has rows).  The
// words are whole aligned 32-bit words, decoded later, so nothing waits on
// them before the state is issued.  No address depends on the state slot:
// at batch 1 the copies then go out while the slot index is still loading.
//
// Row 4 carries dt_bias (a per-head word, read from lane kDtLane) on every
// lane unless `path` is given: then lanes 0-15 fetch the words of the
// pending path entries instead (the fused commit reads them from there).
constexpr int kDtLane = 63;
__device__ __forceinline__ void issue_gates(const dft_verify_args& p, const Item& it, int lane,
                                            uint32_t (*graw)[64], const void* path = nullptr) {
  uint32_t sh;
  const int64_t gi = it.row0 + (lane < it.n ? lane : it.n - 1);
  lds_dma4(word_of(p.a, gi * p.a_row_stride + it.h, p.a_dtype, sh), graw[0]);
  lds_dma4(word_of(p.b, gi * p.b_row_stride + it.h, p.b_dtype, sh), graw[1]);
  // (dense ancestry: the words are not read, any valid source will do)
  const uint32_t* bits = p.anc_bits ? reinterpret_cast<const uint32_t*>(p.anc_bits + gi)
                                    : static_cast<const uint32_t*>(p.y);
  lds_dma4(bits, graw[2]);
  lds_dma4(bits + 1, graw[3]);
  const uint32_t* dt = word_of(p.dt_bias, it.h, p.dt_bias_dtype, sh);
  lds_dma4((path && lane < 16) ? path : static_cast<const void*>(dt), graw[4]);
  lds_dma4(word_of(p.neg_exp_A ? static_cast<const void*>(p.neg_exp_A) : p.A_log, it.h,
                   p.neg_exp_A ? (int)DFT_F32 : p.A_log_dtype, sh),
           graw[5]);
}

// gates of node `lane` from graw (wave 0, lanes < NP): g, beta, ancestry
template <class WK>
__device__ __forceinline__ void decode_gates(const dft_verify_args& p, const Item& it, int lane,
                                             const uint32_t (*graw)[64], WK& wk) {
  uint32_t sha, shb, shdt, shdec;
  const int64_t gi = it.row0 + (lane < it.n ? lane : it.n - 1);
  word_of(p.a, gi * p.a_row_stride + it.h, p.a_dtype, sha);
  word_of(p.b, gi * p.b_row_stride + it.h, p.b_dtype, shb);
  word_of(p.dt_bias, it.h, p.dt_bias_dtype, shdt);
  word_of(p.neg_exp_A ? static_cast<const void*>(p.neg_exp_A) : p.A_log, it.h,
          p.neg_exp_A ? (int)DFT_F32 : p.A_log_dtype, shdec);
  const int i = lane;
  float gv = 0.f, bv = 0.f;
  if (i < it.n) {
    const float a = word_to_f(graw[0][i], sha, p.a_dtype) + word_to_f(graw[4][kDtLane], shdt, p.dt_bias_dtype);
    const float sp = a > 20.f ? a : logf(1.f + expf(fminf(a, 20.f)));
    const uint32_t wdec = graw[5][i];
    const float dec = p.neg_exp_A ? __uint_as_float(wdec) : -expf(word_to_f(wdec, shdec, p.A_log_dtype));
    gv = dec * sp;
    bv = 1.f / (1.f + expf(-word_to_f(graw[1][i], shb, p.b_dtype)));
  }
  wk.gc[i] = gv;
  wk.beta[i] = bv;
  if (p.anc_bits) {
    const uint64_t bits = ((uint64_t)graw[3][i] << 32) | graw[2][i];
    wk.anc[i] = i < it.n ? (bits & mask_upto(i) & mask_below(it.n)) : 0ull;
  }
}

// dense ancestry rows become bit masks (loads and waits right away: only the
// dense form, used by the batch-1 drop-in, takes this path)
template <int NP, int NW, class WK>
__device__ __forceinline__ void dense_ancestry(const dft_verify_args& p, const Item& it, int wave, int lane, WK& wk) {
  const float* ab = p.anc_f32 + (int64_t)it.b * p.anc_req_stride;
  for (int i = wave; i < NP; i += NW) {
    const float v = (i < it.n && lane < it.n) ? ab[i * p.anc_row_stride + lane] : 0.f;
    const uint64_t bits = __ballot(v > 0.5f);
    if (lane == 0) wk.anc[i] = bits & mask_upto(i);
  }
}

// q/k/v rows -> LDS: one 1 KiB copy fills 4 swizzled rows (NP/(4 NW) per wave
// and plane).  Planes M0 .. M1-1 of (q, k, v).  The request has rows.
template <int NP, int M0, int M1, int NW, class RW>
__device__ __forceinline__ void issue_rows(const dft_verify_args& p, const Item& it, int wave, int lane, RW& rw) {
  const int KD = p.hk * kD;
  const int64_t ys = p.y_row_stride;
  const uint16_t* ybase = reinterpret_cast<const uint16_t*>(p.y) + it.row0 * ys;
  const uint16_t* srcs[3] = {ybase + it.hk * kD, ybase + KD + it.hk * kD, ybase + 2 * KD + it.h * kD};
  uint16_t* dsts[3] = {rw.q, rw.k, rw.vrows()};
  const int pc = lane & 15;
#pragma unroll
  for (int u = 0; u < NP / (4 * NW); ++u) {
    const int blk = wave + NW * u;  // rows 4 blk .. 4 blk + 3
    const int i = 4 * blk + (lane >> 4);
    const int isrc = i < it.n ? i : it.n - 1;  // rows past the tree repeat a real row (finite, masked later)
    const int64_t goff = isrc * ys + 8 * ((pc ^ i) & 15);
#pragma unroll
    for (int m = M0; m < M1; ++m) {
      // q and k rows are read again by the k-head's other v-heads (same XCD,
      // same L2); each v row is read once.  Non-temporal v copies measured
      // 1.2% faster at batch 64; non-temporal q/k copies gained nothing.
      const void* src = srcs[m] + goff;
      if (m == 2 && M0 == 2)  // the late v rows, copied alone while Ck computes
        lds_dma16_nt_untracked(src, dsts[m] + 4 * blk * kD);
      else if (m == 2)
        lds_dma16_nt(src, dsts[m] + 4 * blk * kD);
      else
        lds_dma16(src, dsts[m] + 4 * blk * kD);
    }
  }
}

// The whole state tile, group by group (16 16-byte loads per lane).  NT:
// non-temporal loads.  Measured at batch 64 (interleaved runs): the
// read-only verify is 2.9% faster with ordinary loads, the fused commit ->
// verify (which writes the tile back) 0.7% faster with non-temporal ones.
template <bool NT, bool LINES, int NW>
__device__ __forceinline__ void issue_state(const float* S0, int64_t v_stride, int wave, int lane,
                                            f32x4 (&s0r)[Waves<NW>::TT][8]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) issue_state_group<NT, LINES, NW>(S0, v_stride, wave, lane, s, s0r);
}

// x plus lane l ^ 1, l ^ 2 (quad permutes) or l ^ 7 (mirror within the 8
// lanes of a half row): one move each instead of a cross-lane LDS permute
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141;

// 1a: row norms (4 threads per q/k row) and the path-cumulative decay
// (NT / NP = 8 threads per node), spread over all waves.  DPP: the sums over
// a row's 4 threads and a node's 8 are DPP adds, else cross-lane permutes;
// the two give the same sums bit for bit (each step adds a lane's value and
// its partner's, and the 8-lane mirror meets the same quad sums as the
// xor-4 permute), so every kernel's norms and decays agree.  Splitting a
// thread's 16 pair products over 4 accumulators as well was 0.2 us faster
// at batch 1 but rounded the norms differently from the fused kernels,
// whose commit -> verify then no longer matched commit followed by verify.
template <int NP, int NW, bool DPP, class RW, class WK>
__device__ __forceinline__ void phase_norms(const dft_verify_args& p, int tid, const RW& rw, WK& wk) {
  constexpr int NT = Waves<NW>::NT;
  static_assert((2 * NP) % (NT / 4) == 0, "whole passes of q and k rows");
#pragma unroll
  for (int r0 = 0; r0 < 2 * NP; r0 += NT / 4) {
    const int r = r0 + (tid >> 2), qd = tid & 3, i = r % NP;
    const uint16_t* rows = r < NP ? rw.q : rw.k;
    float acc[1] = {0.f};  // bf16 pair dot products, accumulated in fp32
#pragma unroll
    for (int c = 32 * qd; c < 32 * qd + 32; c += 8) {
      const uint4 u = *reinterpret_cast<const uint4*>(rows + qkv_at(i, c));
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bf16x2 v = __builtin_bit_cast(bf16x2, w[e]);
        acc[0] = __builtin_amdgcn_fdot2_f32_bf16(v, v, acc[0], false);
      }
    }
    float ss;
    if constexpr (DPP) {
      ss = acc[0];
      ss = dpp_add<kDppXor1>(ss);
      ss = dpp_add<kDppXor2>(ss);
    } else {
      ss = acc[0];
      ss += __shfl_xor(ss, 1);
      ss += __shfl_xor(ss, 2);
    }
    if (qd == 0) {
      const float rn = rsqrtf(ss + 1e-6f);
      if (r < NP) wk.rq[i] = rn * p.scale;
      else wk.rk[i] = rn;
    }
  }
  constexpr int TPN = NT / NP;  // threads per node, each summing NP / TPN consecutive nodes
  constexpr int JPT = NP / TPN;
  static_assert(JPT % 4 == 0, "whole 16-byte reads of g");
  static_assert(TPN == 8, "the node sums are over 8 lanes");
  const int i = tid / TPN, sub = tid % TPN;
  const uint64_t bits = wk.anc[i];
  float G = 0.f;
#pragma unroll
  for (int q = 0; q < JPT / 4; ++q) {
    const int j0 = sub * JPT + 4 * q;
    const f32x4 g = *reinterpret_cast<const f32x4*>(&wk.gc[j0]);
#pragma unroll
    for (int e = 0; e < 4; ++e) G += ((bits >> (j0 + e)) & 1ull) ? g[e] : 0.f;
  }
  if constexpr (DPP) {
    G = dpp_add<kDppXor1>(G);
    G = dpp_add<kDppXor2>(G);
    G = dpp_add<kDppHalfMirror>(G);  // (each quad's sum plus the other quad's)
  } else {
#pragma unroll
    for (int o = 1; o < TPN; o <<= 1) G += __shfl_xor(G, o);
  }
  if (sub == 0) wk.G[i] = G;
}

// The saves for the commit: normalised keys (once per k-head when saved per
// k-head) and G.  Needs the norms and G; reads the k rows.
// CS: the workgroups of a column split share the saves, each writing key
// columns col0 .. col0 + 128 / CS - 1 (the first one writes G).
// NTS: the threads taking part (tid 0 .. NTS - 1; by default the workgroup).
template <int NP, bool LATE, int NW, class RW, class WK, int CS = 1, int NTS = Waves<NW>::NT>
__device__ __forceinline__ void phase_saves(const VerifyParams& P, const Item& it, int tid, const RW& rw,
                                            const WK& wk, int col0 = 0) {
  constexpr int KQ = 32 / CS;  // 4-column pieces of a key row per workgroup
  static_assert(NTS >= NP, "the G saves take a thread per node");
  const OutArgs p = out_args<LATE>(P);
  const bool per_khead = (p.flags & DFT_VERIFY_AUX_K_PER_KHEAD) != 0;
  if (p.aux_k && (!per_khead || it.rr == 0)) {
    float* dk = p.aux_k + (int64_t)(per_khead ? it.hk : it.h) * p.aux_k_h_stride + it.row0 * p.aux_k_row_stride;
    for (int c = tid; c < it.n * KQ; c += NTS) {
      const int i = c / KQ, d = col0 + (c % KQ) * 4;
      const uint2 u = *reinterpret_cast<const uint2*>(&rw.k[qkv_at(i, d)]);
      const float r = wk.rk[i];
      const f32x4 val = {__uint_as_float(u.x << 16) * r, __uint_as_float(u.x & 0xffff0000u) * r,
                         __uint_as_float(u.y << 16) * r, __uint_as_float(u.y & 0xffff0000u) * r};
      float* dst = dk + i * p.aux_k_row_stride + d;
      if (p.auxk_vec) {
        __builtin_nontemporal_store(val, reinterpret_cast<f32x4*>(dst));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = val[e];
      }
    }
  }
  if (p.aux_g && col0 == 0 && tid < it.n)
    p.aux_g[(int64_t)it.h * p.aux_g_h_stride + (it.row0 + tid) * p.aux_g_row_stride] = wk.G[tid];
}

// 1b/1c: output row scales, the ancestor-masked Gram tiles of A (transposed
// into am) and the diagonal 16x16 blocks of X.  Wave b < NP/16 forms tile
// (b, b) and solves it at once by forward substitution (lane j = column j):
// the solve reads only LDS this wave wrote, and one wave's LDS operations
// are ordered, so no workgroup barrier stands between the two.  The
// off-diagonal tiles follow, spread over the waves.  Pq is formed after the
// off-diagonal levels (phase_pq), in the LDS that A holds until then.
//
// Of X above its diagonal blocks only blocks (b, b + 1), b even, are ever
// read: phase_out's 32-wide k-steps pair block columns 2s and 2s + 1 and skip
// the steps wholly above the diagonal.  Each thread zeroes one element of each.
template <int NP, class RW, class WK>
__device__ __forceinline__ void a_tile(const RW& rw, WK& wk, int ti, int tj, int n16, int g4) {
  constexpr int LDA = WK::LDA;
  const int op = qkv_op8(n16, g4);
  f32x4 acc = {};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const bf16x8 av = *reinterpret_cast<const bf16x8*>(rw.k + 16 * ti * kD + (op ^ (32 * s)));
    const bf16x8 bv = *reinterpret_cast<const bf16x8*>(rw.k + 16 * tj * kD + (op ^ (32 * s)));
    acc = mfma_bf16_16x16x32(av, bv, acc);
  }
  // nodes i0 .. i0 + 3 of this lane: their per-node values in one read each,
  // then selects (no load under a branch), then one 16-byte store
  const int j = 16 * tj + n16, i0 = 16 * ti + 4 * g4;
  const float rkj = wk.rk[j], Gj = wk.G[j];
  const f32x4 bi = *reinterpret_cast<const f32x4*>(&wk.beta[i0]);
  const f32x4 ri = *reinterpret_cast<const f32x4*>(&wk.rk[i0]);
  const f32x4 gi = *reinterpret_cast<const f32x4*>(&wk.G[i0]);
  f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = i0 + r;
    const bool on = ((wk.anc[i] >> j) & 1ull) && j < i;
    const float v = bi[r] * ri[r] * rkj * acc[r] * __expf(gi[r] - Gj);
    out[r] = on ? v : 0.f;
  }
  *reinterpret_cast<f32x4*>(&wk.am()[j * LDA + i0]) = out;
}

// mtn: 16-row tiles that hold nodes (the rest are padding and are skipped);
// KA: rows in flight in the diagonal solves
// WS: the diagonal blocks solved by whole waves (solve_block16_wave), else
// on 16 lanes (solve_block16).
template <int NP, int NW, int KA, bool WS, class RW, class WK>
__device__ __forceinline__ void phase_gram_diag(int tid, const RW& rw, WK& wk, int mtn) {
  constexpr int MT = NP / 16;
  constexpr int LDA = WK::LDA;
  const int lane = tid & 63, wave = tid >> 6, n16 = lane & 15, g4 = lane >> 4;
  if (tid < NP) {
    const float eG = __expf(wk.G[tid]);
    wk.gc[tid] = eG * wk.rk[tid];  // g is no longer needed
    wk.cO[tid] = eG * wk.rq[tid];
  }
  if (wave < mtn) {
    a_tile<NP>(rw, wk, wave, wave, n16, g4);
    if constexpr (WS) {
      solve_block16_wave<LDA, KA>(wk.am(), wk.x(), 16 * wave, lane);
    } else if (lane < 16) {
      const int bb = wave, j = lane;
      float xc[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) xc[i] = (i == j) ? 1.f : 0.f;
      solve_block16<LDA, KA>(xc, wk.am(), 16 * bb);
      materialize16(xc);
#pragma unroll
      for (int i = 0; i < 16; ++i) wk.x()[(16 * bb + i) * LDA + 16 * bb + j] = xc[i];
    }
  }
  int item = 0;
#pragma unroll
  for (int ti = 1; ti < MT; ++ti)
#pragma unroll
    for (int tj = 0; tj < ti; ++tj, ++item)
      // off the waves that solve a diagonal block when there are spare ones
      if (ti < mtn && (NW > MT ? MT + item % (NW - MT) : (MT + item) % NW) == wave) a_tile<NP>(rw, wk, ti, tj, n16, g4);
  if (tid < 256)  // one element of each 16 x 16 block per thread
#pragma unroll
    for (int b = 0; b + 1 < MT; b += 2) wk.x()[(16 * b + (tid >> 4)) * LDA + 16 * (b + 1) + (tid & 15)] = 0.f;
}


// acc + X_(bi, ba) T for T in the accumulator layout, as neg_diag_times
template <int LDA>
__device__ __forceinline__ f32x4 x_block_times(const float* x, int bi, int ba, f32x4 T, f32x4 acc, int n16, int g4) {
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mfma_f32_16x16x4(x[(16 * bi + n16) * LDA + 16 * ba + 4 * g4 + s], T[s], acc);
  return acc;
}

// 1d, one level: off-diagonal blocks X_ij = -D_i sum_{m=j}^{i-1} A_im X_mj at
// distance d = i - j (each level needs the previous ones).  With four block
// rows the last level is folded into the second: the lower-left 2 x 2
// blocks are X_LL = -X_BB A_LL X_TT (X_TT, X_BB the inverses of the
// diagonal 32 x 32 halves, complete after level 1), so
// X_30 = -(X_32 (A_20 X_00 + A_21 X_10) + X_33 (A_30 X_00 + A_31 X_10))
// needs no level-2 block; a third wave forms it beside X_20 and X_31.
// The caller stops after level 2 when MT is 4.
template <int NP, int NW, class WK>
__device__ __forceinline__ void phase_offdiag(int tid, int d, WK& wk, int mtn) {
  constexpr int MT = NP / 16;
  constexpr int LDA = WK::LDA;
  const int lane = tid & 63, wave = tid >> 6, n16 = lane & 15, g4 = lane >> 4;
  const int bj = wave, bi = wave + d;
  if (bi < mtn) {
    f32x4 T = {};
#pragma unroll
    for (int bm = 0; bm < MT; ++bm)
      if (bm >= bj && bm < bi) T = block_mma<LDA, true>(T, wk.am(), bi, bm, wk.x(), bj, n16, g4);
    store_block<LDA>(wk.x(), bi, bj, neg_diag_times<LDA>(wk.x(), bi, T, n16, g4), n16, g4);
  }
  if constexpr (MT == 4) {
    if (d == 2 && wave == 2 && mtn > 3) {
      f32x4 T20 = {}, T30 = {};
#pragma unroll
      for (int bm = 0; bm < 2; ++bm) {
        T20 = block_mma<LDA, true>(T20, wk.am(), 2, bm, wk.x(), 0, n16, g4);
        T30 = block_mma<LDA, true>(T30, wk.am(), 3, bm, wk.x(), 0, n16, g4);
      }
      f32x4 acc = {};
      acc = x_block_times<LDA>(wk.x(), 3, 2, T20, acc, n16, g4);
      acc = x_block_times<LDA>(wk.x(), 3, 3, T30, acc, n16, g4);
      store_block<LDA>(wk.x(), 3, 0, -acc, n16, g4);
    }
  }
}

// Pq(bi, bm): the Gram of the k rows of block bm against the q rows of
// block bi, lane (n, g) holding row 16bi + n at columns 16bm + 4g .. + 3.  The operands are swapped so the
// tile comes out transposed (lane (n, g), element r -> i = 16bi + n,
// j = 16bm + 4g + r), then masked to ancestors-or-self and scaled by
// rq_i rk_j e^{G_i - G_j}.
template <class RW, class WK>
__device__ __forceinline__ f32x4 pq_tile(const RW& rw, const WK& wk, int bi, int bm, int n16, int g4) {
  const int op = qkv_op8(n16, g4);
  f32x4 acc = {};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const bf16x8 kv = *reinterpret_cast<const bf16x8*>(rw.k + 16 * bm * kD + (op ^ (32 * s)));
    const bf16x8 qv = *reinterpret_cast<const bf16x8*>(rw.q + 16 * bi * kD + (op ^ (32 * s)));
    acc = mfma_bf16_16x16x32(kv, qv, acc);
  }
  const int i = 16 * bi + n16, j0 = 16 * bm + 4 * g4;
  const uint64_t ai = wk.anc[i];
  const float rqi = wk.rq[i], Gi = wk.G[i];
  const f32x4 rkj = *reinterpret_cast<const f32x4*>(&wk.rk[j0]);
  const f32x4 gj = *reinterpret_cast<const f32x4*>(&wk.G[j0]);
  f32x4 out;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = rqi * rkj[r] * acc[r] * __expf(Gi - gj[r]);
    out[r] = ((ai >> (j0 + r)) & 1ull) ? v : 0.f;
  }
  return out;
}

// The output products read X and Pq as bf16 hi/lo operand pairs, split once
// here rather than by every wave: in row i, the 32 floats of k-step ks hold
// four 32-byte chunks, chunk g = the 8 hi then the 8 lo halves of columns
// 32ks + 4g .. + 3 and 32ks + 16 + 4g .. + 3 (the order of one MFMA operand),
// so an operand is two 16-byte reads at float 32ks + 8g and 32ks + 8g + 4.
__device__ __forceinline__ void split_bf16x4(f32x4 x, uint2& hi, uint2& lo) {
  const float xs[8] = {x[0], x[1], x[2], x[3], 0.f, 0.f, 0.f, 0.f};
  bf16x8 h, l;
  split_bf16x8(xs, h, l);
  const u32x4 hw = __builtin_bit_cast(u32x4, h), lw = __builtin_bit_cast(u32x4, l);
  hi = uint2{hw[0], hw[1]};
  lo = uint2{lw[0], lw[1]};
}

// 1e: Pq into am, which A no longer needs (the last off-diagonal level has
// read it), in the split operand layout: the blocks (bi, bm <= bi) and the
// zero blocks (b, b + 1), b even, that the output products' 32-wide k-steps
// also read.  Lane (n, g) of tile (bi, bm) holds columns 16bm + 4g .. + 3 of
// row 16bi + n: half bm & 1 of chunk g of k-step bm / 2.  The output takes
// o = cO Cq + Pq vn, which equals cO Cq + M W with M = Pq X because
// vn = X W: the N^3 product M = Pq X is never formed.  Tiles are dealt to
// the waves round robin; rows of padding tiles are skipped.
template <int NP, int NW, class RW, class WK>
__device__ __forceinline__ void phase_pq(int tid, const RW& rw, WK& wk, int mtn) {
  constexpr int MT = NP / 16;
  constexpr int LDA = WK::LDA;
  const int lane = tid & 63, wave = tid >> 6, n16 = lane & 15, g4 = lane >> 4;
  int item = 0;
#pragma unroll
  for (int bi = 0; bi < MT; ++bi) {
    if (bi >= mtn) break;  // padding rows: never read
#pragma unroll
    for (int bm = 0; bm < MT; ++bm) {
      if (bm > bi && (bm != bi + 1 || (bi & 1))) continue;
      if (item++ % NW != wave) continue;
      const f32x4 t = bm <= bi ? pq_tile(rw, wk, bi, bm, n16, g4) : f32x4{};
      uint2 hi, lo;
      split_bf16x4(t, hi, lo);
      float* chunk = &wk.am()[(16 * bi + n16) * LDA + 32 * (bm >> 1) + 8 * g4 + 2 * (bm & 1)];
      *reinterpret_cast<uint2*>(chunk) = hi;
      *reinterpret_cast<uint2*>(chunk + 4) = lo;
    }
  }
}

// 1e': X into the split operand layout, in place.  The 4 lanes of one
// (row, k-step) read its 32 floats before any of them writes (one wave, one
// read instruction before the write: a wave's LDS operations run in order).
// Rows < 32 need k-step 0 only (the products skip the steps wholly above the
// diagonal), rows 32 .. 63 both; rows of padding tiles are skipped.
template <int NP, int NW, class WK>
__device__ __forceinline__ void phase_split_x(int tid, WK& wk, int mtn) {
  constexpr int LDA = WK::LDA;
  constexpr int U0 = 4 * (NP < 32 ? NP : 32);
  constexpr int U = U0 + (NP > 32 ? 8 * (NP - 32) : 0);
  static_assert(U <= Waves<NW>::NT && U0 % 64 == 0, "one unit per thread, whole waves per row range");
  if (tid >= U) return;
  int i, ks;
  if (tid < U0) {
    i = tid >> 2;
    ks = 0;
  } else {
    i = 32 + ((tid - U0) >> 3);
    ks = ((tid - U0) >> 2) & 1;
  }
  const int g = tid & 3;
  if (i >= 16 * mtn) return;
  float* row = wk.x() + i * LDA + 32 * ks;
  float a8[8];
  lds_f32x8_split(row, 4 * g, a8);
  asm volatile("" ::: "memory");  // every lane's reads stay before the writes
  bf16x8 hi, lo;
  split_bf16x8(a8, hi, lo);
  *reinterpret_cast<bf16x8*>(row + 8 * g) = hi;
  *reinterpret_cast<bf16x8*>(row + 8 * g + 4) = lo;
}

// 2: Cq = q_raw S0, Ck = k_raw S0 for the wave's 32 columns.  k-step s, lane
// group g, element e -> k = 32s + 4g + e (e < 4), 32s + 16 + 4g + e-4.  The
// A and B operands of the bf16 MFMA share one lane layout (index lane % 16,
// k = 8 (lane / 16) + e), so swapping them yields the transposed product from
// the same registers: Ck comes out as [node][column] (lane n, g, element r ->
// node 16mt + 4g + r, column 16t + n), Cq as [column][node] (node 16mt + n,
// column 16t + 4g + r), the layout of the output tiles.
// WHICH: 3 = both products, 1 = Cq only, 2 = Ck only (a two-pass form that
// frees the q rows after the first).
// KEEP: 0 = split the state here, 1 = split it here and keep the split in
// sh / sl, 2 = take the split kept by an earlier pass (the two-pass form
// splits once).
template <int NP, int WHICH, int NW, int KEEP, class RW>
__device__ __forceinline__ void phase_cq_ck(int lane, const RW& rw, const f32x4 (&s0r)[Waves<NW>::TT][8],
                                            f32x4 (&cq)[NP / 16][Waves<NW>::TT],
                                            f32x4 (&ck)[NP / 16][Waves<NW>::TT], int mtn,
                                            bf16x8 (&sh)[4][Waves<NW>::TT], bf16x8 (&sl)[4][Waves<NW>::TT]) {
  constexpr int TT = Waves<NW>::TT;
  constexpr int MT = NP / 16;
  constexpr bool DQ = (WHICH & 1) != 0, DK = (WHICH & 2) != 0;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int op = qkv_op4(n16, g4);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if (DQ) cq[mt][t] = f32x4{};
      if (DK) ck[mt][t] = f32x4{};
    }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8 bhi[TT], blo[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if constexpr (KEEP == 2) {
        bhi[t] = sh[s][t];
        blo[t] = sl[s][t];
      } else {
        const float xs[8] = {s0r[t][2 * s][0],     s0r[t][2 * s][1],     s0r[t][2 * s][2],     s0r[t][2 * s][3],
                             s0r[t][2 * s + 1][0], s0r[t][2 * s + 1][1], s0r[t][2 * s + 1][2], s0r[t][2 * s + 1][3]};
        split_bf16x8(xs, bhi[t], blo[t]);
        if constexpr (KEEP == 1) {
          sh[s][t] = bhi[t];
          sl[s][t] = blo[t];
        }
      }
    }
    const int o1 = op ^ (32 * s), o2 = op ^ (32 * s + 16);  // columns 32s + 4g .., 32s + 16 + 4g ..
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt >= mtn) break;  // padding rows stay zero
      bf16x8 aq{}, ak{};
      if (DQ) aq = lds_bf16x8_split(rw.q + 16 * mt * kD + o1, rw.q + 16 * mt * kD + o2);
      if (DK) ak = lds_bf16x8_split(rw.k + 16 * mt * kD + o1, rw.k + 16 * mt * kD + o2);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        if (DQ) cq[mt][t] = mfma_bf16_16x16x32(bhi[t], aq, cq[mt][t]);
        if (DK) ck[mt][t] = mfma_bf16_16x16x32(ak, bhi[t], ck[mt][t]);
        if (DQ) cq[mt][t] = mfma_bf16_16x16x32(blo[t], aq, cq[mt][t]);
        if (DK) ck[mt][t] = mfma_bf16_16x16x32(ak, blo[t], ck[mt][t]);
      }
    }
  }
}

// 3a: W = beta (v - e^G rk Ck) in the accumulator layout, split into bf16
// hi/lo B operands: k-step ks, lane group g, element e -> node 32ks + 4g + e
// (e < 4), 32ks + 16 + 4g + e-4, i.e. registers of tiles 2ks, 2ks+1.
// NW here counts column waves (waves x column split); col0: the workgroup's
// first value column.
template <int NP, int NW, class RW, class WK>
__device__ __forceinline__ void phase_w(int lane, int wave, const RW& rw, const WK& wk,
                                        const f32x4 (&ck)[NP / 16][Waves<NW>::TT],
                                        bf16x8 (&wh)[NP / 32][Waves<NW>::TT], bf16x8 (&wl)[NP / 32][Waves<NW>::TT],
                                        int col0 = 0) {
  constexpr int TT = Waves<NW>::TT, CW = Waves<NW>::CW;
  constexpr int KS = NP / 32;
  const int n16 = lane & 15, g4 = lane >> 4;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    // beta and e^G rk of nodes 16mt + 4g .. + 3, mt = 2ks, 2ks + 1
    f32x4 bt[2], gcv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bt[h] = *reinterpret_cast<const f32x4*>(&wk.beta[16 * (2 * ks + h) + 4 * g4]);
      gcv[h] = *reinterpret_cast<const f32x4*>(&wk.gc[16 * (2 * ks + h) + 4 * g4]);
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int col = col0 + CW * wave + 16 * t + n16;
      float w8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int h = e >> 2, mt = 2 * ks + h, r = e & 3;
        const int i = 16 * mt + 4 * g4 + r;
        const float vv = bf16_bits_to_f32(rw.vrows()[qkv_at(i, col)]);
        w8[e] = bt[h][r] * (vv - gcv[h][r] * ck[mt][t][r]);
      }
      split_bf16x8(w8, wh[ks][t], wl[ks][t]);
    }
  }
}

// 3b: vn = X W, then o = cO Cq + Pq vn.  Both products are computed
// transposed, the left factor (W, then vn) as the A operand, so lane (n, g)
// holds node 16mt + n at the four consecutive columns 16t + 4g .. +3: one
// 16-byte (vn) or 8-byte (o) write each.  vn always goes to its staging rows
// in the (then free) q/k region, from which each wave reads its own columns
// back in W's operand layout; vn and o leave through LDS when the flags
// allow, else they are stored directly.
template <int NP, int NW, class RW, class WK>
__device__ __forceinline__ void phase_out(const VerifyParams& P, const Item& it, int lane, int wave, RW& rw,
                                          const WK& wk, const f32x4 (&cq)[NP / 16][Waves<NW>::TT],
                                          const bf16x8 (&wh)[NP / 32][Waves<NW>::TT],
                                          const bf16x8 (&wl)[NP / 32][Waves<NW>::TT], int mtn, int col0 = 0) {
  constexpr int TT = Waves<NW>::TT, CW = Waves<NW>::CW;
  constexpr int MT = NP / 16;
  constexpr int KS = NP / 32;
  constexpr int LDA = WK::LDA;
  const dft_verify_args& p = P.a;
  const int n16 = lane & 15, g4 = lane >> 4;
  float* vn_s = reinterpret_cast<float*>(rw.q);  // spans q and k
  uint16_t* o_s = rw.ostage();
  // tile mt of [F; V] (F = X or Pq in the split operand layout, V = W or
  // vn): lane (n, g) gets node 16mt + n
  auto product = [&](const float* f, const bf16x8 (&vh)[KS][TT], const bf16x8 (&vl)[KS][TT], int mt, f32x4 (&acc)[TT]) {
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = f32x4{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (32 * ks > 16 * mt + 15) continue;  // both factors are lower triangular
      const float* chunk = f + (16 * mt + n16) * LDA + 32 * ks + 8 * g4;
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(chunk);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(chunk + 4);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        acc[t] = mfma_bf16_16x16x32(vh[ks][t], ah, acc[t]);
        acc[t] = mfma_bf16_16x16x32(vl[ks][t], ah, acc[t]);
        acc[t] = mfma_bf16_16x16x32(vh[ks][t], al, acc[t]);
      }
    }
  };
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (mt >= mtn) break;  // padding rows: not stored
    f32x4 acc[TT];
    product(wk.x(), wh, wl, mt, acc);
    const int i = 16 * mt + n16;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int col = col0 + CW * wave + 16 * t + 4 * g4;
      *reinterpret_cast<f32x4*>(&vn_s[vn_at(i, col)]) = acc[t];
      if (!P.vn_stage && p.aux_v && i < it.n) {
        float* dst = p.aux_v + (int64_t)it.h * p.aux_v_h_stride + (it.row0 + i) * p.aux_v_row_stride + col;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = acc[t][r];
      }
    }
  }
  // vn back in W's layout (k-step ks, lane (n, g), element e -> node
  // 32ks + 4g + e (e < 4), 32ks + 16 + 4g + e-4; column 16t + n), the wave's
  // own columns only (its LDS writes are ordered before these reads).  Rows
  // of the tree's last tile past the tree are exact zeros (beta = 0 there,
  // so W and vn are), and Pq is zero in their columns; padding tiles were
  // never written and are replaced by zeros.  With i = 32ks + 16h + 4g + r,
  // vn_at(i, c) = 4g kD + (c & 3) + (32ks + 16h + r) kD + (lane chunk ^ (16h + r)) * 4.
  bf16x8 vh[KS][TT], vl[KS][TT];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int col = col0 + CW * wave + 16 * t + n16;
      const float* base = vn_s + 4 * g4 * kD + (col & 3);
      const int ch = ((col >> 2) ^ (4 * g4)) & 31;
      float v8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int h = e >> 2, r = e & 3;
        const float v = base[(32 * ks + 16 * h + r) * kD + ((ch ^ (16 * h + r)) << 2)];
        v8[e] = 2 * ks + h < mtn ? v : 0.f;  // uniform
      }
      split_bf16x8(v8, vh[ks][t], vl[ks][t]);
    }
  // the late-v form stages o in x: every wave must be done with X first
  if constexpr (RW::kLateV) __syncthreads();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if (mt >= mtn) break;
    f32x4 acc[TT];
    product(wk.am(), vh, vl, mt, acc);
    const int i = 16 * mt + n16;
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int col = col0 + CW * wave + 16 * t + 4 * g4;
      const f32x4 ov = wk.cO[i] * cq[mt][t] + acc[t];
      if (P.o_stage) {
        const bf16x2 lo = __builtin_convertvector((f32x2{ov[0], ov[1]}), bf16x2);  // round to nearest even
        const bf16x2 hi = __builtin_convertvector((f32x2{ov[2], ov[3]}), bf16x2);
        uint2 w;
        __builtin_memcpy(&w.x, &lo, 4);
        __builtin_memcpy(&w.y, &hi, 4);
        *reinterpret_cast<uint2*>(&o_s[qkv_at(i, col)]) = w;
      } else if (i < it.n) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          st_f(p.o, (it.row0 + i) * p.o_row_stride + (int64_t)it.h * p.o_h_stride + col + r, p.o_dtype, ov[r]);
      }
    }
  }
}

// 3c: staged vn and o as whole 16-byte row pieces.  All outputs (these and
// the key saves) are written once and not read back by this launch: they go
// out as non-temporal stores, which at batch 64 made the verify 6.6% and the
// fused commit -> verify 3.1% faster than ordinary stores.
// CS: value columns split over CS workgroups; this one stores columns col0 ..
// col0 + 128 / CS - 1 of every row.
template <int NP, bool LATE, int NW, class RW, int CS = 1>
__device__ __forceinline__ void phase_stores(const VerifyParams& P, const Item& it, int tid, const RW& rw,
                                             int col0 = 0) {
  constexpr int NT = Waves<NW>::NT;
  constexpr int VQ = 32 / CS, OQ = 16 / CS;  // 16-byte pieces of a row per workgroup
  const OutArgs p = out_args<LATE>(P);
  const float* vn_s = reinterpret_cast<const float*>(rw.q);
  const uint16_t* o_s = rw.ostage();
  if (p.vn_stage) {  // rows of 32 x 16 bytes
    float* dst = p.aux_v + (int64_t)it.h * p.aux_v_h_stride + it.row0 * p.aux_v_row_stride;
#pragma unroll
    for (int u = 0; u < NP * VQ / NT; ++u) {
      const int i = (NT / VQ) * u + tid / VQ, q = col0 / 4 + tid % VQ;
      if (i < it.n)
        __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(&vn_s[vn_at(i, 4 * q)]),
                                    reinterpret_cast<f32x4*>(dst + i * p.aux_v_row_stride + 4 * q));
    }
  }
  if (p.o_stage) {  // rows of 16 x 16 bytes
    uint16_t* dst = static_cast<uint16_t*>(p.o) + it.row0 * p.o_row_stride + (int64_t)it.h * p.o_h_stride;
#pragma unroll
    for (int u = 0; u < NP * OQ / NT; ++u) {
      const int i = (NT / OQ) * u + tid / OQ, q = col0 / 8 + tid % OQ;
      if (i < it.n)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&o_s[qkv_at(i, 8 * q)]),
                                    reinterpret_cast<u32x4*>(dst + i * p.o_row_stride + 8 * q));
    }
  }
}

// The fused kernel's status word (wave 0 of the request's head-0
// workgroup), written at the end of the workgroup from this lane's pending
// path entry word (still in gate row 4 of LDS there), the entries' ancestry
// rows (walk, where issue_walk_dma copied them; nothing is read from it when
// nothing was pending) and the arguments re-read from the kernel-argument
// segment.  Evaluated early and held through the state stream, the flags
// cost the kernel a spilled register.
__device__ __forceinline__ void fused_status(const Item& it, int lane, uint32_t path_word, const uint32_t* walk) {
  typedef const __attribute__((address_space(4))) VerifyParams* KParams;
  KParams kp = (KParams)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(kp));
  int32_t* status = kp->a.status;
  if (!status) return;
  const int b = it.b;
  const int32_t* cu = kp->a.cu_seqlens;
  const int nn = kp->a.n_nodes;
  const int span = cu ? cu[b + 1] - cu[b] : nn;
  PendingHead ph = pending_head(&kp->c, b);
  // no slot of its own: nothing is committed, as in the commit itself
  if (kp->a.state_indices && ld_i(kp->a.state_indices, b, kp->a.state_indices_dtype) < 0) ph.len = 0;
  const Pending pd = decode_pending(ph, lane, path_word);
  const bool walk_bad = kp->c.prev_anc_bits && pd.last >= 0 && !pending_walk_ok(pd, lane, walk, ph.bound);
  if (lane == 0)
    status[b] = (span < 0 || span > nn ? DFT_STATUS_SPAN : 0) | (pd.bad ? DFT_STATUS_PATH : 0) |
                (walk_bad ? DFT_STATUS_WALK : 0);
}

// The body of the one-head-per-workgroup kernels (COMMIT: the fused commit ->
// verify form).
// CS (plain verify of up to 32 nodes): the item's value columns are split
// over CS workgroups, CS items apart in the grid's last dimension; each
// forms phase 1 in full and phases 2-3 on its 128 / CS columns.
// ---------------------------------------------------------------------------
// Trees of 33-64 nodes in small launches: each (request, v-head) runs on two
// workgroups of 8 waves, each taking 64 value columns (col0 = 0 or 64).  Both
// form phase 1 in full.  In phases 2-3 wave w takes column tile c = w & 3
// (16 columns) and half h = w >> 2: it reads rows k = 64h .. 64h + 63 of its
// columns' state (so a workgroup reads its 32 KiB once) and forms partial Cq
// and Ck over those k for every node tile.  The two halves of a column tile
// swap the partials of each other's node tiles through LDS, and from then on
// wave (c, h) owns node tiles 2h and 2h + 1: their W, vn and o.  X W and
// Pq vn of tiles 2-3 also need k-step 0 (nodes 0-31), whose W and vn the
// first half passes on through LDS.  The sums of the two k halves are formed
// in another order than the one-workgroup kernel's, so Cq and Ck can differ
// from it in the last bits.
// ---------------------------------------------------------------------------
template <bool ON>
struct HalfXch {
  int unused;
};
template <>
struct HalfXch<true> {
  f32x4 part[8][4][64];  // wave w's partials of its partner's node tiles: Cq, Cq, Ck, Ck
  bf16x8 w[4][2][64];    // the first half's W (k-step 0; hi, lo) of column tile c
};

// An item chosen by the caller (the mixed-width kernel): the request (its
// class-relative index when records are read) and v-head, the class bounds
// item_rows applies, and where the item's arrays start in mixed_lds.
struct Given {
  Item it;
  int n_lo, n_hi, cls;
  int lds_off;
};

// k-step s (rows k = 32s .. 32s + 31) of column tile c's state, in the MFMA layout
__device__ __forceinline__ void issue_state_half(const float* S0, int64_t v_stride, int c, int lane, int s,
                                                 f32x4& a, f32x4& b) {
  const int n16 = lane & 15, g4 = lane >> 4;
  const float* rowp = S0 + (int64_t)(16 * c + n16) * v_stride + 4 * g4 + 32 * s;
  a = *reinterpret_cast<const f32x4*>(rowp);
  b = *reinterpret_cast<const f32x4*>(rowp + 16);
}

// partial Cq / Ck over k-steps 2h, 2h + 1 for every node tile, in
// phase_cq_ck's layouts (WHICH and KEEP as there; s0h holds the two k-steps)
template <int WHICH, int KEEP, class RW>
__device__ __forceinline__ void cq_ck_half(int lane, int h, const RW& rw, const f32x4 (&s0h)[4], f32x4 (&cq)[4],
                                           f32x4 (&ck)[4], int mtn, bf16x8 (&sh)[2], bf16x8 (&sl)[2]) {
  constexpr bool DQ = (WHICH & 1) != 0, DK = (WHICH & 2) != 0;
  const int n16 = lane & 15, g4 = lane >> 4;
  const int op = qkv_op4(n16, g4);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    if (DQ) cq[mt] = f32x4{};
    if (DK) ck[mt] = f32x4{};
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int s = 2 * h + j;
    bf16x8 bhi, blo;
    if constexpr (KEEP == 2) {
      bhi = sh[j];
      blo = sl[j];
    } else {
      const float xs[8] = {s0h[2 * j][0],     s0h[2 * j][1],     s0h[2 * j][2],     s0h[2 * j][3],
                           s0h[2 * j + 1][0], s0h[2 * j + 1][1], s0h[2 * j + 1][2], s0h[2 * j + 1][3]};
      split_bf16x8(xs, bhi, blo);
      if constexpr (KEEP == 1) {
        sh[j] = bhi;
        sl[j] = blo;
      }
    }
    const int o1 = op ^ (32 * s), o2 = op ^ (32 * s + 16);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (mt >= mtn) break;  // padding rows stay zero
      bf16x8 aq{}, ak{};
      if (DQ) aq = lds_bf16x8_split(rw.q + 16 * mt * kD + o1, rw.q + 16 * mt * kD + o2);
      if (DK) ak = lds_bf16x8_split(rw.k + 16 * mt * kD + o1, rw.k + 16 * mt * kD + o2);
      if (DQ) cq[mt] = mfma_bf16_16x16x32(bhi, aq, cq[mt]);
      if (DK) ck[mt] = mfma_bf16_16x16x32(ak, bhi, ck[mt]);
      if (DQ) cq[mt] = mfma_bf16_16x16x32(blo, aq, cq[mt]);
      if (DK) ck[mt] = mfma_bf16_16x16x32(ak, blo, ck[mt]);
    }
  }
}

// Phases 2-3 of the two-workgroup 64-wide form, from the state's k half s0h
// to o and vn staged (or stored) for node tiles 2h, 2h + 1 of the wave's 16
// columns.  Starts after phase 1 (X and Pq split, no barrier yet).
template <class RW, class WK>
__device__ __forceinline__ void tail_halves(const VerifyParams& P, const Item& it, int lane, int wave, RW& rw,
                                            const WK& wk, HalfXch<true>& xc, const f32x4 (&s0h)[4], int mtn,
                                            int col0) {
  constexpr int LDA = WK::LDA;
  const dft_verify_args& p = P.a;
  const int c = wave & 3, h = wave >> 2, n16 = lane & 15, g4 = lane >> 4;
  // Cq first; once every wave is done with the q rows, the v rows are
  // copied into their region while Ck computes (as in the one-workgroup form)
  f32x4 cq[4], ck[4];
  bf16x8 sh[2], sl[2];
  cq_ck_half<1, 1>(lane, h, rw, s0h, cq, ck, mtn, sh, sl);
  __syncthreads();  // X and Pq complete, the q rows consumed
  issue_rows<64, 2, 3, 8>(p, it, wave, lane, rw);
  cq_ck_half<2, 2>(lane, h, rw, s0h, cq, ck, mtn, sh, sl);
  // the partner's node tiles go to it; this wave keeps tiles 2h, 2h + 1
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    xc.part[wave][j][lane] = h ? cq[j] : cq[2 + j];
    xc.part[wave][2 + j][lane] = h ? ck[j] : ck[2 + j];
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));  // the v row copies (untracked by the backend)
  __syncthreads();
  const int pw = wave ^ 4;
  f32x4 cqo[2], cko[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    cqo[j] = (h ? cq[2 + j] : cq[j]) + xc.part[pw][j][lane];
    cko[j] = (h ? ck[2 + j] : ck[j]) + xc.part[pw][2 + j][lane];
  }
  // W = beta (v - e^G rk Ck) of k-step h (node tiles 2h, 2h + 1), in
  // phase_w's operand layout
  const int colw = col0 + 16 * c + n16;
  bf16x8 wh, wl;
  {
    f32x4 bt[2], gcv[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      bt[hh] = *reinterpret_cast<const f32x4*>(&wk.beta[16 * (2 * h + hh) + 4 * g4]);
      gcv[hh] = *reinterpret_cast<const f32x4*>(&wk.gc[16 * (2 * h + hh) + 4 * g4]);
    }
    float w8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int hh = e >> 2, r = e & 3;
      const int i = 16 * (2 * h + hh) + 4 * g4 + r;
      const float vv = bf16_bits_to_f32(rw.vrows()[qkv_at(i, colw)]);
      w8[e] = bt[hh][r] * (vv - gcv[hh][r] * cko[hh][r]);
    }
    split_bf16x8(w8, wh, wl);
  }
  if (h == 0) {
    xc.w[c][0][lane] = wh;
    xc.w[c][1][lane] = wl;
  }
  __syncthreads();  // every wave has read its v rows (the q/k region takes vn); W of k-step 0 is out
  bf16x8 w0h = wh, w0l = wl;
  if (h) {
    w0h = xc.w[c][0][lane];
    w0l = xc.w[c][1][lane];
  }
  // tile mt of [F; V] (F = X or Pq in the split operand layout, V = W or vn
  // of k-steps 0 and 1): lane (n, g) gets node 16mt + n, columns 4g .. + 3
  auto product = [&](const float* f, bf16x8 v0h, bf16x8 v0l, bf16x8 v1h, bf16x8 v1l, int mt) {
    f32x4 acc{};
    {
      const float* chunk = f + (16 * mt + n16) * LDA + 8 * g4;
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(chunk);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(chunk + 4);
      acc = mfma_bf16_16x16x32(v0h, ah, acc);
      acc = mfma_bf16_16x16x32(v0l, ah, acc);
      acc = mfma_bf16_16x16x32(v0h, al, acc);
    }
    if (h) {  // tiles 2-3: k-step 1 too (uniform); both factors are lower triangular
      const float* chunk = f + (16 * mt + n16) * LDA + 32 + 8 * g4;
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(chunk);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(chunk + 4);
      acc = mfma_bf16_16x16x32(v1h, ah, acc);
      acc = mfma_bf16_16x16x32(v1l, ah, acc);
      acc = mfma_bf16_16x16x32(v1h, al, acc);
    }
    return acc;
  };
  float* vn_s = reinterpret_cast<float*>(rw.q);  // spans q and k
  const int colo = col0 + 16 * c + 4 * g4;      // the product tiles' first column
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int mt = 2 * h + j;
    if (mt >= mtn) break;  // padding rows: not stored (uniform)
    const f32x4 acc = product(wk.x(), w0h, w0l, wh, wl, mt);
    const int i = 16 * mt + n16;
    *reinterpret_cast<f32x4*>(&vn_s[vn_at(i, colo)]) = acc;
    if (!P.vn_stage && p.aux_v && i < it.n) {
      float* dst = p.aux_v + (int64_t)it.h * p.aux_v_h_stride + (it.row0 + i) * p.aux_v_row_stride + colo;
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[r] = acc[r];
    }
  }
  // vn of every tile staged; every wave is done with X, where o is staged
  __syncthreads();
  // vn back in W's layout (phase_out's read-back) for k-steps 0 and, in the
  // second half, 1; padding tiles were never written and read as zeros
  bf16x8 vh[2], vl[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const float* base = vn_s + 4 * g4 * kD + (colw & 3);
    const int ch = ((colw >> 2) ^ (4 * g4)) & 31;
    float v8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int hh = e >> 2, r = e & 3;
      const float v = base[(32 * ks + 16 * hh + r) * kD + ((ch ^ (16 * hh + r)) << 2)];
      v8[e] = (2 * ks + hh < mtn && ks <= h) ? v : 0.f;  // uniform
    }
    split_bf16x8(v8, vh[ks], vl[ks]);
  }
  uint16_t* o_s = rw.ostage();
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int mt = 2 * h + j;
    if (mt >= mtn) break;
    const f32x4 acc = product(wk.am(), vh[0], vl[0], vh[1], vl[1], mt);
    const int i = 16 * mt + n16;
    const f32x4 ov = wk.cO[i] * cqo[j] + acc;
    if (P.o_stage) {
      const bf16x2 lo = __builtin_convertvector((f32x2{ov[0], ov[1]}), bf16x2);  // round to nearest even
      const bf16x2 hi = __builtin_convertvector((f32x2{ov[2], ov[3]}), bf16x2);
      uint2 w;
      __builtin_memcpy(&w.x, &lo, 4);
      __builtin_memcpy(&w.y, &hi, 4);
      *reinterpret_cast<uint2*>(&o_s[qkv_at(i, colo)]) = w;
    } else if (i < it.n) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        st_f(p.o, (it.row0 + i) * p.o_row_stride + (int64_t)it.h * p.o_h_stride + colo + r, p.o_dtype, ov[r]);
    }
  }
}

// The kernel arguments the plain verify reads before its first copies,
// forced into scalar registers at entry: read where they are used, behind
// the branches on item_rows' index arrays, they came in some eight
// dependent rounds of scalar loads, which a latency-bound launch (batch 1)
// waits out one by one (batch-1 verify 8.35 -> 8.17 us at 32 nodes, 12.05
// -> 11.72 at 64).  Only the column-split kernels, which serve the small
// launches, do so: after the opaque statement the index arrays are read
// with vector loads, which in a full launch queue behind the state stream
// (the ragged layer measured 112.1 -> 113.5 us with it).
__device__ __forceinline__ void args_early(const VerifyParams& P) {
  const dft_verify_args& p = P.a;
  asm volatile("" ::"s"(p.batch), "s"(p.n_nodes), "s"(p.hk), "s"(p.hv), "s"(p.y), "s"(p.y_row_stride),
               "s"(p.cu_seqlens), "s"(p.a), "s"(p.a_row_stride), "s"(p.a_dtype), "s"(p.b), "s"(p.b_row_stride),
               "s"(p.b_dtype), "s"(p.A_log), "s"(p.A_log_dtype));
  asm volatile("" ::"s"(p.dt_bias), "s"(p.dt_bias_dtype), "s"(p.neg_exp_A), "s"(p.anc_f32), "s"(p.anc_bits),
               "s"(p.state), "s"(p.state_slot_stride), "s"(p.state_h_stride), "s"(p.state_v_stride),
               "s"(p.state_indices), "s"(p.state_indices_dtype), "s"(p.status), "s"(p.size_order), "s"(P.n_lo),
               "s"(P.n_hi), "s"(P.cls));
}

// tid_in: the thread within the item's waves; blk: the block id the item is
// taken from.  With GIVEN the item and its LDS come from `given`.
template <int NP, bool S0VEC, bool COMMIT, bool RAWK, bool RVN, bool PDMA = false, int CS = 1, bool GIVEN = false>
__device__ __forceinline__ void verify_body(const VerifyParams& P, int tid_in, int blk, const Given& given) {
  constexpr int MT = NP / 16;
  constexpr int NW = WavesFor<NP>();
  // the 64-wide column split: waves split the k half and node tiles (tail_halves)
  constexpr bool kHalves = NP > 32 && CS > 1;
  constexpr int NWC = kHalves ? NW : NW * CS;  // column waves of the item (of all its workgroups)
  constexpr int TT = Waves<NWC>::TT, CW = Waves<NWC>::CW;
  static_assert(CS == 1 || !COMMIT, "the column split serves the plain verify");
  static_assert(!kHalves || (CS == 2 && S0VEC), "the 64-wide split takes two workgroups and a vector state");
  // The 32-wide fused form runs phase 1 (which needs no state) before its
  // commit, under the state stream, and stages the commit's keys and
  // write-back in the v region, whose rows it copies in afterwards.
  constexpr bool kEarly = COMMIT && !VerifySmem<NP>::kLateV;
  constexpr int kPlanes = (VerifySmem<NP>::kLateV || kEarly) ? 2 : 3;  // the late forms copy v rows later
  // PDMA: the path's raw rows are copied into LDS ahead of the state tile
  // (16-byte aligned key and value rows; issue_path_dma)
  constexpr bool kPathDma = PDMA;
  static_assert(!PDMA || (kEarly && RVN && RAWK), "the path copies serve the 32-wide recompute form");
  constexpr int kQkvDma = kPlanes * (NP / (4 * NW));          // row copies per wave
  constexpr int kStateLoads = 8 * TT, kGroupLoads = 2 * TT;   // per lane: whole tile, one k-step group
  const dft_verify_args& p = P.a;
  static_assert(!GIVEN || (!COMMIT && CS == 1), "a given item is a plain verify");
  // the verify's arrays: the body's own, or (a given item) its region of mixed_lds
  VerifySmem<NP>& sm = [&]() -> VerifySmem<NP>& {
    if constexpr (GIVEN) {
      return *reinterpret_cast<VerifySmem<NP>*>(reinterpret_cast<char*>(mixed_lds) + given.lds_off);
    } else {
      __shared__ VerifySmem<NP> own;
      return own;
    }
  }();
  // the recomputed path values' matrices and key norms: only the forms that
  // recompute them hold them (4.3 KiB)
  float* const rvx = [&]() -> float* {
    if constexpr (GIVEN) {
      return nullptr;
    } else {
      __shared__ alignas(16) float own[RVN ? kRvx : 4];
      return own;
    }
  }();

  // (the wave index as a scalar: in a vector register it is held, and at the
  // fused form's register cap spilled, through phase 1)
  const int tid = tid_in, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n16 = lane & 15, g4 = lane >> 4;

  if constexpr (!COMMIT && CS > 1) args_early(P);
  Item it;
  int col0 = 0;  // the workgroup's first value column
  if constexpr (GIVEN) {
    it = given.it;
  } else if constexpr (CS > 1) {
    const int items = p.batch * p.hv;
    const int sp = (unsigned)blk / (unsigned)items;  // (uniform)
    col0 = sp * (kD / CS);
    item_heads(p, blk - sp * items, it);
  } else {
    item_heads(p, blk, it);
  }
  if (!item_rows<NP>(p, it, GIVEN ? given.n_lo : P.n_lo, GIVEN ? given.n_hi : P.n_hi, GIVEN ? given.cls : P.cls))
    return;
  // Thread 0 of the request's head-0 workgroup writes its status word (the
  // condition is evaluated where it is written: held from here, it would
  // cost the fused kernel a register through the state stream).
  if constexpr (!COMMIT)
    if (p.status && it.h == 0 && col0 == 0 && tid == 0) p.status[it.b] = it.span_bad ? DFT_STATUS_SPAN : 0;
  // (the state rows of the workgroup's columns: v is the row index)
  const float* S0 = CS > 1 ? it.S0 + (int64_t)col0 * p.state_v_stride : it.S0;
  PendingHead ph{};
  if constexpr (COMMIT) {
    ph = pending_head(&P.c, it.b);
    if (it.no_slot) ph.len = 0;  // no slot of its own: nothing is committed
    if (it.n == 0) {  // nothing to verify this step: the commit alone
      const uint32_t word = *path_word(P.c, it.b, lane);
      Pending pd = decode_pending(ph, lane, word);
      uint32_t* walk = sm.graw[4];
      if (pd.last >= 0) {  // uniform (one request)
        f32x4 s0r[TT][8];
        PathKeys<NW, RAWK> kr;
        PathVals<NW, RVN> pv;
        // (the ancestry rows go first: the keys the commit waits for land behind them)
        issue_walk_dma<false>(P.c, pd, wave, lane, S0, walk);
        issue_state<true, kEarly, NW>(S0, p.state_v_stride, wave, lane, s0r);
        issue_pending<NW, RAWK, RVN>(P.c, pd, it.h, wave, lane, S0, kr, pv);
        commit_tile<NW, kEarly, RAWK, RVN>(pd, sm.pkey(), rvx, kr, pv, wave, lane, s0r,
                                           P.c.prev_anc_bits ? walk : nullptr, ph.bound);
        __syncthreads();  // every wave has read the staged keys: am + x take the write-back staging
        if (pd.last >= 0)  // uniform: a path that is not a walk was dropped
          store_state<NW>(const_cast<float*>(S0), p.state_v_stride, wave, lane, s0r, sm.amx + wave * 512);
      }
      if (it.h == 0 && wave == 0) fused_status(it, lane, word, walk);
      return;
    }
  }
  if (it.n == 0) return;

  // ---- 0. issue order (vector memory returns in order): the gates and
  // ancestry bits (wave 0), the q/k/v rows straight into LDS, then the 64 KiB
  // state tile into registers.  Phase 1 only waits for what precedes the
  // state; the state keeps streaming underneath it.
  // (fused form: the pending path's entry words travel in gate row 4)
  // 64-wide fused form: every wave loads the previous step's path entry words
  // first, decodes them as soon as they land (the gate and row copies issued
  // behind them need not have) and issues the path's keys, values and gains
  // ahead of the state tile, so that they are in when the tile is.  (The
  // 32-wide form issues them after phase 1: held in registers through phase 1
  // beside the tile, they would be spilled.)
  Pending pd{};
  PathKeys<NW, RAWK> kr;
  PathVals<NW, RVN> pv;
  uint32_t pword = 0;
  if constexpr (COMMIT && !kEarly) pword = *path_word(P.c, it.b, lane);
  if constexpr (kPathDma) {
    pword = *path_word(P.c, it.b, lane);
    asm volatile("" ::: "memory");
  }
  if (wave == 0) issue_gates(p, it, lane, sm.graw, COMMIT ? path_word(P.c, it.b, lane) : nullptr);
  if (p.anc_f32) dense_ancestry<NP, NW>(p, it, wave, lane, sm);
  issue_rows<NP, 0, kPlanes, NW>(p, it, wave, lane, sm);
  if constexpr (COMMIT && !kEarly) {
    pd = decode_pending(ph, lane, pword);
    issue_pending<NW, RAWK, RVN>(P.c, pd, it.h, wave, lane, S0, kr, pv);
    issue_walk_dma<false>(P.c, pd, wave, lane, S0, sm.graw[4]);  // (lands before the state, as the gates)
  }
  if constexpr (kPathDma) {
    const Pending pd0 = decode_pending(ph, lane, pword);
    issue_path_dma<NW>(P.c, pd0, it.h, wave, lane, S0, reinterpret_cast<uint16_t*>(sm.vrows()), rvx);
    issue_walk_dma<false>(P.c, pd0, wave, lane, S0, sm.graw[4]);
  }
  asm volatile("" ::: "memory");

  f32x4 s0r[TT][8];
  f32x4 s0h[4];  // the 64-wide split: k-steps 2h, 2h + 1 of the wave's column tile
  // The verify issues its state tile in 4 groups (the k-steps phase 2
  // consumes in order) through phase 1: a wave blocked on a full memory queue
  // then stalls between compute phases instead of ahead of all of them
  // (1.7% faster at batch 64).  So does the 32-wide fused form, whose commit
  // follows phase 1 (64.05 -> 62.01 us at batch 64, raw rows copied ahead of
  // the tile), except the form that holds raw path rows in registers beside
  // the tile, which spilled; the 64-wide one commits before phase 1 and
  // issues its tile at once.
  constexpr bool kSplit = S0VEC && (!COMMIT || (kEarly && (kPathDma || !(RAWK && RVN))));
  if constexpr (kHalves) {
    issue_state_half(S0, p.state_v_stride, wave & 3, lane, 2 * (wave >> 2), s0h[0], s0h[1]);
  } else if (kSplit) {
    issue_state_group<COMMIT, kEarly, NWC>(S0, p.state_v_stride, wave, lane, 0, s0r);
  } else if (S0VEC) {
    issue_state<COMMIT, kEarly, NWC>(S0, p.state_v_stride, wave, lane, s0r);
  } else {
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s0r[t][j][e] = S0[(int64_t)(CW * wave + 16 * t + n16) * p.state_v_stride +
                            (int64_t)(16 * j + 4 * g4 + e) * p.state_k_stride];
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));  // element loads: no overlap on this path
  }
  asm volatile("" ::: "memory");

  if (wave == 0) {
    // the gate words were wave 0's first copies: wait for them only (the
    // fused form: for everything before the state, the path loads included)
    __builtin_amdgcn_s_waitcnt(waitcnt_imm((COMMIT ? 0 : kQkvDma) + (kSplit ? kGroupLoads : kStateLoads), 15));
    asm volatile("" ::: "memory");
    if (lane < NP) decode_gates(p, it, lane, sm.graw, sm);
  }
  // Wait for the row loads and gates (everything issued before the state),
  // then make the LDS writes of all waves visible.  A plain __syncthreads()
  // here would also drain the state loads.
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(kSplit ? kGroupLoads : kStateLoads, 0));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  // 64-wide fused form: the norms overlap the state stream.  As soon as the
  // tile has landed the path is committed into it (keys staged in am + x,
  // still unused) and the tile goes back to its slot, so that the write-back
  // streams under the rest of phase 1.
  phase_norms<NP, NW, (NP > 32 || CS > 1)>(p, tid, sm, sm);
  __syncthreads();
  if constexpr (COMMIT && !kEarly) {
    commit_tile<NW, false, RAWK, RVN>(pd, sm.pkey(), rvx, kr, pv, wave, lane, s0r,
                                      P.c.prev_anc_bits ? sm.graw[4] : nullptr, ph.bound);
    // everything this wave loaded has been consumed: no load is left in
    // flight past the (conditional) write-back
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
    if (pd.last >= 0) {  // uniform over the workgroup (one request)
      __syncthreads();  // every wave has read the staged keys: am + x take the write-back staging
      store_state<NW>(const_cast<float*>(S0), p.state_v_stride, wave, lane, s0r, sm.amx + wave * 512);
    }
    __syncthreads();  // am and x take the Gram tiles and X
  }
  if constexpr (kHalves)
    issue_state_half(S0, p.state_v_stride, wave & 3, lane, 2 * (wave >> 2) + 1, s0h[2], s0h[3]);
  else if constexpr (kSplit)
    issue_state_group<COMMIT, kEarly, NWC>(S0, p.state_v_stride, wave, lane, 1, s0r);
  // (the 32-wide fused form saves after Cq/Ck: at this point its tile is
  // still streaming in, and the saves' stores would wait on the full queue)
  // The saves go to the waves past the diagonal blocks, which form only
  // off-diagonal A tiles while the others solve (the 64-wide kernel: waves
  // 4-7; the 32-wide: waves 2-3).
  constexpr int kSaveWave0 = MT;
  const int mtn = (it.n + 15) >> 4;  // uniform over the workgroup
  // (the plain verify with a vector state has registers for 3 rows ahead.
  // The 32-wide fused forms, whose phase 1 runs under their state stream,
  // keep the 16-lane solve: with the whole-wave one the headline form
  // measured 62.73 -> 63.13 us at batch 64, and the form holding raw path
  // rows in registers spilled.)
  constexpr bool kWaveSolve = !kEarly;
  phase_gram_diag<NP, NW, (!COMMIT && S0VEC) ? 3 : 1, kWaveSolve>(tid, sm, sm, mtn);
  if constexpr (!kEarly)
    if (wave >= kSaveWave0)
      phase_saves<NP, COMMIT, NW, VerifySmem<NP>, VerifySmem<NP>, CS, 64 * (NW - kSaveWave0)>(
          P, it, tid - 64 * kSaveWave0, sm, sm, col0);
  if constexpr (kEarly && RVN) {
    // The recompute forms hold few registers for the path (raw rows, 10 per
    // lane): their loads go out here, once the diagonal solves (a 32-float
    // column per lane) are done, and stream in under the rest of phase 1
    // (65.4 -> 65.0 us at batch 64; issued before the solves they spilled).
    pd = decode_pending(ph, lane, sm.graw[4][lane & 15]);
    if constexpr (!kPathDma) {
      issue_walk_dma<true>(P.c, pd, wave, lane, S0, sm.graw[4]);  // ahead of the path loads that cover it
      issue_pending<NW, RAWK, RVN>(P.c, pd, it.h, wave, lane, S0, kr, pv);
    }
  }
  if constexpr (kSplit && !kHalves) issue_state_group<COMMIT, kEarly, NWC>(S0, p.state_v_stride, wave, lane, 2, s0r);
  __syncthreads();
#pragma unroll
  for (int d = 1; d < (MT == 4 ? 3 : MT); ++d) {  // (four block rows: level 3 is folded into level 2)
    if (d >= mtn) break;
    phase_offdiag<NP, NW>(tid, d, sm, mtn);
    __syncthreads();
  }
  if constexpr (kSplit && !kHalves) issue_state_group<COMMIT, kEarly, NWC>(S0, p.state_v_stride, wave, lane, 3, s0r);
  phase_pq<NP, NW>(tid, sm, sm, mtn);
  phase_split_x<NP, NW>(tid, sm, mtn);
  if constexpr (kEarly) {
    // the path's entry words came with the gates (row 4); the saved-value
    // forms' loads go out now, so that they are not held in registers through
    // phase 1
    if constexpr (!RVN) {
      pd = decode_pending(ph, lane, sm.graw[4][lane & 15]);
      issue_walk_dma<true>(P.c, pd, wave, lane, S0, sm.graw[4]);
      issue_pending<NW, RAWK, RVN>(P.c, pd, it.h, wave, lane, S0, kr, pv);
    }
    float* stage = reinterpret_cast<float*>(sm.vrows());  // 8 KiB: the 16 path keys, then the write-back
    if constexpr (kPathDma)
      path_from_lds<NW>(P.c, pd, it.h, wave, lane, reinterpret_cast<const uint16_t*>(stage), rvx, kr, pv);
    commit_tile<NW, true, RAWK, RVN, kPathDma>(pd, stage, rvx, kr, pv, wave, lane, s0r,
                                               P.c.prev_anc_bits ? sm.graw[4] : nullptr, ph.bound);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
    if (pd.last >= 0) {  // uniform over the workgroup (one request)
      __syncthreads();  // every wave has read the staged keys
      store_state<NW>(const_cast<float*>(S0), p.state_v_stride, wave, lane, s0r, stage + wave * 512);
    }
    __syncthreads();  // every wave has read its staging back: the v region takes the v rows
    // (row addresses recomputed from an opaque copy of the lane id: shared
    // with the q/k copies at the start, they would be held through the commit)
    int lane_v = lane;
    asm volatile("" : "+v"(lane_v));
    issue_rows<NP, 2, 3, NW>(p, it, wave, lane_v, sm);
  }

  f32x4 cq[MT][TT], ck[MT][TT];
  if constexpr (kHalves) {
    // the 64-wide split's exchange between the two halves (40 KiB)
    __shared__ HalfXch<true> xch;
    tail_halves(P, it, lane, wave, sm, sm, xch, s0h, mtn, col0);
  } else if constexpr (VerifySmem<NP>::kLateV) {
    // Cq first; once every wave is done with the q rows, the v rows are
    // copied into their region while Ck computes
    bf16x8 sh[4][TT], sl[4][TT];  // the state split once, for both passes
    phase_cq_ck<NP, 1, NWC, 1>(lane, sm, s0r, cq, ck, mtn, sh, sl);
    __syncthreads();  // X and Pq complete, the q rows consumed
    issue_rows<NP, 2, 3, NW>(p, it, wave, lane, sm);
    phase_cq_ck<NP, 2, NWC, 2>(lane, sm, s0r, cq, ck, mtn, sh, sl);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));  // the v row copies (untracked by the backend)
    __syncthreads();
  } else {
    bf16x8 sh[4][TT], sl[4][TT];  // (unused: one pass)
    phase_cq_ck<NP, 3, NWC, 0>(lane, sm, s0r, cq, ck, mtn, sh, sl);
    if constexpr (kEarly) __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));  // the v row copies (untracked)
    __syncthreads();  // X and Pq complete
  }
  if constexpr (kEarly) phase_saves<NP, COMMIT, NW>(P, it, tid, sm, sm);  // the k rows are intact until phase 3
  if constexpr (!kHalves) {
    bf16x8 wh[NP / 32][TT], wl[NP / 32][TT];
    phase_w<NP, NWC>(lane, wave, sm, sm, ck, wh, wl, col0);
    __syncthreads();  // every wave has read its v rows: the q/k/v region takes the outputs
    phase_out<NP, NWC>(P, it, lane, wave, sm, sm, cq, wh, wl, mtn, col0);
  }
  if (P.vn_stage || P.o_stage) {
    __syncthreads();
    // fused form: an opaque thread id, so that the store offsets are
    // recomputed here instead of held (and spilled) from phase 1
    int tid_s = tid;
    if constexpr (COMMIT) asm volatile("" : "+v"(tid_s));
    phase_stores<NP, COMMIT, NW, VerifySmem<NP>, CS>(P, it, tid_s, sm, col0);
  }
  if constexpr (COMMIT)
    if (it.h == 0 && wave == 0) fused_status(it, lane, sm.graw[4][lane & 15], sm.graw[4]);
}

// Both widths run at 4 waves per SIMD (at most 128 registers): the 32-wide
// kernel as 4 workgroups of 4 waves per CU, the 64-wide one as 2 of 8 waves
// (its LDS holds two per CU).  The 64-wide column split holds one workgroup
// per CU (its LDS), 2 waves per SIMD.
template <int NP, bool S0VEC, int CS = 1>
__global__ void __launch_bounds__(64 * WavesFor<NP>())
    __attribute__((amdgpu_waves_per_eu((NP > 32 && CS > 1) ? 2 : 4))) tree_verify_kernel(const VerifyParams P) {
  verify_body<NP, S0VEC, false, false, false, false, CS>(P, threadIdx.x, blockIdx.x, Given{});
}

// A packed batch with trees on both sides of 32 nodes and size-order records,
// in one launch of 8-wave workgroups (2 per CU: the LDS of one 64-wide item
// or of two 32-wide ones).  Blocks [0, c1 Hv) take the (request, v-head)
// items of the c1 requests over 32 nodes on the 64-wide body; each block
// after them takes v-heads 2j and 2j + 1 of one of the c0 other requests,
// one per half of the workgroup (4 waves each) on the 32-wide body.  The two
// halves verify the same tree (same node count, same exits), so they pass the
// same barriers.  The 64-wide class's last generation then shares the chip
// with the small trees instead of leaving most of it idle in front of a
// second kernel.
// Records of another launch shape are ignored: block b then takes item b
// and its request's size picks the body; a small tree's v-heads 2j, 2j + 1
// go to the block of head 2j, and the other block exits.  Either way every
// item runs the body of its size class, as in the two-kernel launch.
template <bool S0VEC>
__global__ void __launch_bounds__(64 * WavesFor<64>()) __attribute__((amdgpu_waves_per_eu(4)))
tree_verify_mixed_kernel(const VerifyParams P) {
  const dft_verify_args& p = P.a;
  const int4 hd = reinterpret_cast<const int4*>(p.size_order)[0];
  const bool rec = hd.z == p.n_nodes && hd.w == p.batch;  // uniform
  const int blk = blockIdx.x, half = threadIdx.x >> 8, R = p.hv / p.hk;
  Given g;
  g.n_lo = INT_MIN;
  g.n_hi = INT_MAX;
  g.lds_off = 0;
  bool wide;
  if (rec) {
    const int c0 = hd.x, c1 = hd.y, hp = p.hv >> 1;
    wide = blk < c1 * p.hv;
    if (wide) {
      item_heads(p, c1, blk, g.it);  // q < c1: the class-1 records from the back
      g.cls = 1;
    } else {
      const int j = blk - c1 * p.hv;
      if (j >= c0 * hp) return;
      g.it.b = j / hp;
      g.it.h = 2 * (j - g.it.b * hp);
      g.cls = 0;
    }
  } else {
    item_heads(p, blk, g.it);
    const int span = p.cu_seqlens[g.it.b + 1] - p.cu_seqlens[g.it.b];
    wide = span > 32;  // (cut to n_nodes, which is over 32 here)
    if (!wide && (g.it.h & 1)) return;
    g.cls = -1;
    if (wide) g.n_lo = 33;
  }
  if (wide) {
    verify_body<64, S0VEC, false, false, false, false, 1, true>(P, threadIdx.x, blk, g);
  } else {
    g.it.h += half;
    g.it.hk = g.it.h / R;
    g.it.rr = g.it.h - g.it.hk * R;
    g.n_hi = 32;
    g.lds_off = half * (int)sizeof(VerifySmem<32>);
    verify_body<32, S0VEC, false, false, false, false, 1, true>(P, threadIdx.x & 255, blk, g);
  }
}

// P must stay this kernel's first (only) argument: out_args<true> reads it
// back from offset 0 of the kernel-argument segment.
static_assert(std::is_trivially_copyable<VerifyParams>::value, "VerifyParams is passed by value to the kernels");
// RAWK: the pending keys are the previous step's raw bf16 rows; RVN: the
// path's values are recomputed from raw rows; PDMA: (32-wide, both raw)
// those rows are copied into LDS ahead of the state tile
template <int NP, bool RAWK, bool RVN, bool PDMA = false>
__global__ void __launch_bounds__(64 * WavesFor<NP>()) __attribute__((amdgpu_waves_per_eu(4)))
tree_commit_verify_kernel(const VerifyParams P) {
  verify_body<NP, true, true, RAWK, RVN, PDMA>(P, threadIdx.x, blockIdx.x, Given{});
}

static VerifyParams make_params(const dft_verify_args* a) {
  VerifyParams P;
  P.a = *a;
  P.c = dft_pending_commit{};
  const uintptr_t sp = reinterpret_cast<uintptr_t>(a->state);
  P.s0_vec = a->state_k_stride == 1 && (sp % 16) == 0 && (a->state_v_stride % 4) == 0 &&
             (a->state_h_stride % 4) == 0 && (a->state_slot_stride % 4) == 0;
  P.auxk_vec = a->aux_k && (reinterpret_cast<uintptr_t>(a->aux_k) % 16) == 0 && (a->aux_k_row_stride % 4) == 0 &&
               (a->aux_k_h_stride % 4) == 0;
  P.vn_stage = a->aux_v && (reinterpret_cast<uintptr_t>(a->aux_v) % 16) == 0 && (a->aux_v_row_stride % 4) == 0 &&
               (a->aux_v_h_stride % 4) == 0;
  P.o_stage = a->o_dtype == DFT_BF16 && (reinterpret_cast<uintptr_t>(a->o) % 16) == 0 && (a->o_row_stride % 8) == 0 &&
              (a->o_h_stride % 8) == 0;
  P.n_lo = INT_MIN;
  P.n_hi = INT_MAX;
  P.cls = -1;
  return P;
}

// A packed batch whose largest tree exceeds 32 nodes is split by tree size:
// the 64-wide kernel (two workgroups per CU: its LDS and registers) takes the
// requests of 33-64 nodes and the 32-wide kernel (four per CU) the rest, each
// exiting at once on the other's requests.  The sizes stay on the device.
// The 64-wide kernel goes first: the reverse order measured 0.4% slower on
// 128 requests of 8-64 nodes.  With size-order records each kernel takes its
// own class's requests from the front of its grid, and its exiting blocks
// come last.  The plain verify with records, a vector state and an even
// v-head count runs instead as the one mixed-width kernel
// (tree_verify_mixed_kernel): 112.98 -> 111.65 and 112.12 -> 110.28 us per
// ragged layer in interleaved runs on two boxes.
static void split_by_size(const dft_verify_args* a, const VerifyParams& P, VerifyParams& narrow, VerifyParams& wide,
                          bool& split) {
  narrow = wide = P;
  split = a->cu_seqlens != nullptr && a->n_nodes > 32;
  if (split) {
    narrow.n_hi = 32;
    wide.n_lo = 33;
    if (a->size_order) {
      narrow.cls = 0;
      wide.cls = 1;
    }
  }
}

// Requests by size class (dft_size_order): one workgroup, chunks of 1024
// requests; per chunk each wave counts its classes by ballot, and the block
// adds the counts of the waves before it.  Class 0 (at most 32 nodes) fills
// records 0, 1, .. and class 1 records batch - 1, batch - 2, .., both in
// request order; the header holds the two counts, n_nodes and batch.
__global__ void __launch_bounds__(1024) size_order_kernel(const int32_t* cu, int batch, int n_nodes, int4* order) {
  __shared__ int counts[16][2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int done_small = 0, done_large = 0;
  for (int c0 = 0; c0 < batch; c0 += 1024) {
    const int i = c0 + tid;
    const bool in = i < batch;
    const int row0 = in ? cu[i] : 0;
    const int span = in ? cu[i + 1] - row0 : 0;
    const int n = span < 0 ? 0 : (span > n_nodes ? n_nodes : span);
    const bool small = in && n <= 32, large = in && n > 32;
    const uint64_t bs = __ballot(small), bl = __ballot(large);
    const uint64_t below = (1ull << lane) - 1ull;
    if (lane == 0) {
      counts[wave][0] = __popcll(bs);
      counts[wave][1] = __popcll(bl);
    }
    __syncthreads();
    int off_s = 0, off_l = 0, tot_s = 0, tot_l = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      const int cs = counts[w][0], cl = counts[w][1];
      off_s += w < wave ? cs : 0;
      off_l += w < wave ? cl : 0;
      tot_s += cs;
      tot_l += cl;
    }
    const int4 rec = make_int4(i, row0, span, 0);
    if (small) order[1 + done_small + off_s + __popcll(bs & below)] = rec;
    if (large) order[batch - (done_large + off_l + __popcll(bl & below))] = rec;
    done_small += tot_s;
    done_large += tot_l;
    __syncthreads();  // counts is rewritten by the next chunk
  }
  if (tid == 0) order[0] = make_int4(done_small, done_large, n_nodes, batch);
}

int launch_size_order(const int32_t* cu_seqlens, int batch, int n_nodes, int32_t* order, hipStream_t stream) {
  hipLaunchKernelGGL(size_order_kernel, dim3(1), dim3(1024), 0, stream, cu_seqlens, batch, n_nodes,
                     reinterpret_cast<int4*>(order));
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

// Launches of up to 32 nodes whose items would leave most of the chip idle
// (at most kSplitItems of them: batch 1 at 32 v-heads is 32) split each
// item's value columns over two workgroups: each forms phase 1 in full and
// phases 2-3, the state read and the stores on half the columns, which
// shortens a workgroup's life where the launch is latency-bound.
// Launches over 32 nodes with at most kSplitItems64 items do the same with
// the 64-wide kernel (tail_halves; 110 KiB of LDS, one workgroup per CU, so
// at most 256 workgroups for the 256 CUs).
constexpr int kSplitItems = 256, kSplitItems64 = 128;

int launch_tree_verify(const dft_verify_args* a, hipStream_t stream) {
  const VerifyParams P = make_params(a);
  const dim3 grid((unsigned)(a->batch * a->hv)), block(64 * WavesFor<32>()), block64(64 * WavesFor<64>());
  VerifyParams narrow, wide;
  bool split;
  split_by_size(a, P, narrow, wide, split);
  const int64_t items = (int64_t)a->batch * a->hv;
  if (a->n_nodes > 32 && items <= kSplitItems64 && P.s0_vec) {
    const dim3 grid2((unsigned)(2 * items));
    hipLaunchKernelGGL((tree_verify_kernel<64, true, 2>), grid2, block64, 0, stream, wide);
    if (split) hipLaunchKernelGGL((tree_verify_kernel<32, true, 2>), grid2, block, 0, stream, narrow);
    return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
  }
  if (a->n_nodes <= 32 && items <= kSplitItems) {
    const dim3 grid2((unsigned)(2 * items));
    if (P.s0_vec)
      hipLaunchKernelGGL((tree_verify_kernel<32, true, 2>), grid2, block, 0, stream, narrow);
    else
      hipLaunchKernelGGL((tree_verify_kernel<32, false, 2>), grid2, block, 0, stream, narrow);
    return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
  }
  if (split && a->size_order && P.s0_vec && a->hv % 2 == 0) {
    hipLaunchKernelGGL((tree_verify_mixed_kernel<true>), grid, block64, 0, stream, P);
    return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
  }
  if (a->n_nodes > 32) {
    if (P.s0_vec)
      hipLaunchKernelGGL((tree_verify_kernel<64, true>), grid, block64, 0, stream, wide);
    else
      hipLaunchKernelGGL((tree_verify_kernel<64, false>), grid, block64, 0, stream, wide);
  }
  if (a->n_nodes <= 32 || split) {
    if (P.s0_vec)
      hipLaunchKernelGGL((tree_verify_kernel<32, true>), grid, block, 0, stream, narrow);
    else
      hipLaunchKernelGGL((tree_verify_kernel<32, false>), grid, block, 0, stream, narrow);
  }
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

// The caller has checked that the state takes 16-byte accesses.
int launch_tree_commit_verify(const dft_verify_args* a, const dft_pending_commit* c, hipStream_t stream) {
  VerifyParams P = make_params(a);
  P.c = *c;
  const dim3 grid((unsigned)(a->batch * a->hv)), block(64 * WavesFor<32>()), block64(64 * WavesFor<64>());
  VerifyParams narrow, wide;
  bool split;
  split_by_size(a, P, narrow, wide, split);
  // the previous step's raw key rows, recomputed values (validated by the caller)
  const int form = (c->keys == nullptr ? 1 : 0) + (c->values == nullptr ? 2 : 0);
  // both as raw rows whose 16-byte pieces are aligned: the 32-wide kernel
  // copies them into LDS ahead of the state tile
  const auto al16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
  const bool pdma = form == 3 && al16(c->key_rows) && al16(c->value_rows) && c->kr_h_stride % 8 == 0 &&
                    c->kr_row_stride % 8 == 0 && c->vr_h_stride % 8 == 0 && c->vr_row_stride % 8 == 0;
#define DFT_FUSED(np, g, b, prm)                                                                               \
  switch (form) {                                                                                              \
    case 0: hipLaunchKernelGGL((tree_commit_verify_kernel<np, false, false>), g, b, 0, stream, prm); break;   \
    case 1: hipLaunchKernelGGL((tree_commit_verify_kernel<np, true, false>), g, b, 0, stream, prm); break;    \
    case 2: hipLaunchKernelGGL((tree_commit_verify_kernel<np, false, true>), g, b, 0, stream, prm); break;    \
    default: hipLaunchKernelGGL((tree_commit_verify_kernel<np, true, true>), g, b, 0, stream, prm); break;    \
  }
  if (a->n_nodes > 32) DFT_FUSED(64, grid, block64, wide)
  if (a->n_nodes <= 32 || split) {
    if (pdma)
      hipLaunchKernelGGL((tree_commit_verify_kernel<32, true, true, true>), grid, block, 0, stream, narrow);
    else
      DFT_FUSED(32, grid, block, narrow)
  }
#undef DFT_FUSED
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// standalone in-place (I+A)^-1 (fc1_block_inverse.py): one wave per matrix,
// lane j solves (I+A) x = e_j by forward substitution with column j in registers.
// ---------------------------------------------------------------------------
template <int NP>
__global__ void __launch_bounds__(64) block_inverse_kernel(float* x, int n, int64_t mat_stride) {
  constexpr int LD = NP + 4;
  __shared__ float at[NP * LD];  // at[m][i] = A[i][m], strict lower part only
  float* m = x + (int64_t)blockIdx.x * mat_stride;
  const int lane = threadIdx.x;
  if (lane < NP)
    for (int mm = 0; mm < NP; ++mm)
      at[mm * LD + lane] = (lane < n && mm < n && mm < lane) ? m[lane * n + mm] : 0.f;
  __syncthreads();
  float c0[32], c1[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    c0[i] = (i == lane) ? 1.f : 0.f;
    c1[i] = (i + 32 == lane) ? 1.f : 0.f;
  }
  solve_block32<LD>(c0, at, 0);
  materialize32(c0);
  if constexpr (NP == 64) {
    update_block32<LD>(c1, c0, at, 0, 32);
    solve_block32<LD>(c1, at, 32);
    materialize32(c1);
  }
  __syncthreads();
  if (lane < n) {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if (i < n) m[i * n + lane] = c0[i];
    if constexpr (NP == 64) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        if (i + 32 < n) m[(i + 32) * n + lane] = c1[i];
    }
  }
}

int launch_block_inverse(float* x, int n_mats, int n, int64_t mat_stride, hipStream_t stream) {
  if (n <= 32)
    hipLaunchKernelGGL(block_inverse_kernel<32>, dim3(n_mats), dim3(64), 0, stream, x, n, mat_stride);
  else
    hipLaunchKernelGGL(block_inverse_kernel<64>, dim3(n_mats), dim3(64), 0, stream, x, n, mat_stride);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
