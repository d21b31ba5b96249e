// Fused GDN tree verify for gfx950: one workgroup (4 wave64) per
// (request, v-head) does prepare + (I+A)^-1 + finish of
// tree_kernels.py:135-208 in a single pass over the recurrent state.
//
// Math (per head; q_n, k_n normalised, rq/rk the row scales, so that
// q_n = rq * q_raw and k_n = rk * k_raw with q_raw/k_raw exact bf16):
//   G_i   = sum_{j anc-or-self i} g_j
//   A_ij  = [j strict anc i] beta_i (k_n,i . k_n,j) e^{G_i - G_j}
//   Cq    = q_raw S0,  Ck = k_raw S0                   (bf16 MFMA, S0 split hi+lo)
//   (I+A) vn = diag(beta) (v - diag(e^G rk) Ck)        (= X(beta v) - X(beta e^G k) S0, :182-186)
//   o     = diag(e^G rq) Cq + Pq vn,  Pq_ij = [j anc-or-self i] (q_n,i . k_n,j) e^{G_i-G_j}
//
// Work split: wave w owns the 32 value columns [32w, 32w+32).
//  * The 64 KiB state is streamed once, straight into MFMA B operands of
//    v_mfma_f32_16x16x32_bf16: lane (n = l%16, g = l/16) loads 16 bytes at
//    k = 16j + 4g of state row n, so the 4 lanes of a row cover a whole 64-byte
//    sector per instruction.  The contraction order over k is chosen to match
//    (a permutation of k applied to both operands).  Only S0 needs the hi/lo
//    split: the left operands are the exact raw bf16 q/k rows.
//  * The triangular solve runs with one lane per value column holding the
//    whole column in registers (forward substitution, no cross-lane traffic,
//    a dependency chain of N steps); the ancestor structure only enters
//    through A.  X = (I+A)^-1 is never formed.
//  * o accumulates in the 16x16 accumulator layout of phase 2 (fp32 MFMA for
//    Pq vn), so Cq never leaves registers.
#include "dft_device.h"

namespace dft {

constexpr int kD = 128;
constexpr int kQS = kD + 8;  // LDS row stride (bf16) of q/k/v rows: 272 B

struct VerifyParams {
  dft_verify_args a;
  int s0_vec;    // state rows 16-byte aligned with k stride 1
  int auxk_vec;  // aux_k rows 16-byte aligned
};

template <int NP>
struct VerifySmem {
  static constexpr int LDA = NP + 4;  // fp32 row pitch, rows 16-byte aligned
  union {
    struct {
      uint16_t q[NP * kQS];
      uint16_t k[NP * kQS];
    } qk;                    // raw q/k rows (phases 1-2)
    float ct[4][32 * LDA];   // per wave: Ck, then vn, transposed to [column][node]
  } u;
  uint16_t v[NP * kQS];
  float cqs[NP == 64 ? 4 * 32 * LDA : 1];  // 64-node trees: Cq parked across the solve
  float at[NP * LDA];  // at[m][i] = A[i][m]
  float pq[NP * LDA];  // pq[i][m]
  float g[NP], G[NP], eG[NP], beta[NP], rq[NP], rk[NP];
  uint64_t anc[NP];
};

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

// 8 bf16 of one LDS row as two 8-byte halves at columns c0 and c0 + 16
__device__ __forceinline__ bf16x8 lds_bf16x8_split(const uint16_t* row, int c0) {
  const uint2 lo = *reinterpret_cast<const uint2*>(row + c0);
  const uint2 hi = *reinterpret_cast<const uint2*>(row + c0 + 16);
  const uint4 w = {lo.x, lo.y, hi.x, hi.y};
  return __builtin_bit_cast(bf16x8, w);
}

template <int NP>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NP == 32 ? 4 : 1))) tree_verify_kernel(const VerifyParams P) {
  constexpr int MT = NP / 16;  // 16-node tiles
  constexpr int LDA = VerifySmem<NP>::LDA;
  const dft_verify_args& p = P.a;
  __shared__ VerifySmem<NP> sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n16 = lane & 15, g4 = lane >> 4;

  // ---- block -> (request b, v-head h); the R v-heads sharing a k-head get
  // block ids 8 apart so that they land on the same XCD (shared q/k in L2).
  const int R = p.hv / p.hk;
  const int pairs = p.batch * p.hk;
  const int full = (pairs / 8) * 8 * R;
  const int id = blockIdx.x;
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
  const int b = pair / p.hk, hk = pair - b * p.hk, h = hk * R + rr;

  int64_t row0;
  int n;
  if (p.cu_seqlens) {
    row0 = p.cu_seqlens[b];
    n = p.cu_seqlens[b + 1] - p.cu_seqlens[b];
  } else {
    row0 = (int64_t)b * p.n_nodes;
    n = p.n_nodes;
  }
  n = n < 0 ? 0 : (n > NP ? NP : n);
  if (n == 0) return;

  int64_t slot = b;
  if (p.state_indices) {
    slot = ld_i(p.state_indices, b, p.state_indices_dtype);
    if (slot < 0) slot = 0;
  }
  const float* S0 = p.state + slot * p.state_slot_stride + (int64_t)h * p.state_h_stride;

  // ---- 1. state loads first.  s0r[t][j] holds S0[k = 16j + 4g + e][v = 32w + 16t + n]
  f32x4 s0r[2][8];
  if (P.s0_vec) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float* rowp = S0 + (int64_t)(32 * wave + 16 * t + n16) * p.state_v_stride + 4 * g4;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        s0r[t][j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(rowp + 16 * j));
    }
  } else {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s0r[t][j][e] = S0[(int64_t)(32 * wave + 16 * t + n16) * p.state_v_stride +
                            (int64_t)(16 * j + 4 * g4 + e) * p.state_k_stride];
  }

  const int KD = p.hk * kD;
  const int64_t ys = p.y_row_stride;
  const uint16_t* ybase = reinterpret_cast<const uint16_t*>(p.y) + row0 * ys;

  // ---- 2. raw q/k/v rows to LDS (16-byte loads, rows >= n zero-filled)
  {
    const uint16_t* yq = ybase + hk * kD;
    const uint16_t* yk = yq + KD;
    const uint16_t* yv = ybase + 2 * KD + h * kD;
    for (int c = tid; c < NP * 16; c += 256) {
      const int i = c >> 4, ch = (c & 15) * 8;
      uint4 vq = {0u, 0u, 0u, 0u}, vk = vq, vv = vq;
      if (i < n) {
        vq = *reinterpret_cast<const uint4*>(yq + i * ys + ch);
        vk = *reinterpret_cast<const uint4*>(yk + i * ys + ch);
        vv = *reinterpret_cast<const uint4*>(yv + i * ys + ch);
      }
      *reinterpret_cast<uint4*>(&sm.u.qk.q[i * kQS + ch]) = vq;
      *reinterpret_cast<uint4*>(&sm.u.qk.k[i * kQS + ch]) = vk;
      *reinterpret_cast<uint4*>(&sm.v[i * kQS + ch]) = vv;
    }
  }
  // ---- 3. gates and ancestry
  if (tid < NP) {
    const int i = tid;
    float gi = 0.f, bi = 0.f;
    if (i < n) {
      const float a = ld_f(p.a, (row0 + i) * p.a_row_stride + h, p.a_dtype) +
                      ld_f(p.dt_bias, h, p.dt_bias_dtype);
      const float sp = a > 20.f ? a : logf(1.f + expf(fminf(a, 20.f)));
      const float dec = p.neg_exp_A ? p.neg_exp_A[h] : -expf(ld_f(p.A_log, h, p.A_log_dtype));
      gi = dec * sp;
      const float bb = ld_f(p.b, (row0 + i) * p.b_row_stride + h, p.b_dtype);
      bi = 1.f / (1.f + expf(-bb));
    }
    sm.g[i] = gi;
    sm.beta[i] = bi;
    if (p.anc_bits) sm.anc[i] = i < n ? (p.anc_bits[row0 + i] & mask_upto(i) & mask_below(n)) : 0ull;
  }
  if (p.anc_f32) {
    const float* ab = p.anc_f32 + (int64_t)b * p.anc_req_stride;
    for (int i = wave; i < NP; i += 4) {
      const float v = (i < n && lane < n) ? ab[i * p.anc_row_stride + lane] : 0.f;
      const uint64_t bits = __ballot(v > 0.5f);
      if (lane == 0) sm.anc[i] = bits & mask_upto(i);
    }
  }
  __syncthreads();

  // ---- 4. row norms and path-cumulative decay
  if (tid < 2 * NP) {
    const uint16_t* rowp = (tid < NP ? sm.u.qk.q : sm.u.qk.k) + (tid % NP) * kQS;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kD; c += 8) {
      const uint4 u = *reinterpret_cast<const uint4*>(rowp + c);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = __uint_as_float(w[e] << 16), hi = __uint_as_float(w[e] & 0xffff0000u);
        ss += lo * lo + hi * hi;
      }
    }
    const float r = rsqrtf(ss + 1e-6f);
    if (tid < NP) sm.rq[tid] = r * p.scale;
    else sm.rk[tid - NP] = r;
  } else if (tid < 3 * NP) {
    const int i = tid - 2 * NP;
    const uint64_t bits = sm.anc[i];
    float G = 0.f;
#pragma unroll
    for (int j = 0; j < NP; ++j)
      if ((bits >> j) & 1ull) G += sm.g[j];
    sm.G[i] = G;
    sm.eG[i] = __expf(G);
  }
  __syncthreads();

  // ---- 5. saves for the commit (normalised keys, G) and the Gram tiles:
  // lower 16x16 tiles of k k^T (-> A, stored transposed) and q k^T (-> Pq)
  const bool per_khead = (p.flags & DFT_VERIFY_AUX_K_PER_KHEAD) != 0;
  if (p.aux_k && (!per_khead || rr == 0)) {
    float* dk = p.aux_k + (int64_t)(per_khead ? hk : h) * p.aux_k_h_stride + row0 * p.aux_k_row_stride;
    for (int c = tid; c < n * 32; c += 256) {
      const int i = c >> 5, d = (c & 31) * 4;
      const uint2 u = *reinterpret_cast<const uint2*>(&sm.u.qk.k[i * kQS + d]);
      const float r = sm.rk[i];
      const f32x4 val = {__uint_as_float(u.x << 16) * r, __uint_as_float(u.x & 0xffff0000u) * r,
                         __uint_as_float(u.y << 16) * r, __uint_as_float(u.y & 0xffff0000u) * r};
      float* dst = dk + i * p.aux_k_row_stride + d;
      if (P.auxk_vec) {
        *reinterpret_cast<f32x4*>(dst) = val;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e] = val[e];
      }
    }
  }
  if (p.aux_g && tid < n) p.aux_g[(int64_t)h * p.aux_g_h_stride + (row0 + tid) * p.aux_g_row_stride] = sm.G[tid];
  {
    int item = 0;
#pragma unroll
    for (int which = 0; which < 2; ++which)
#pragma unroll
      for (int it = 0; it < MT; ++it)
#pragma unroll
        for (int jt = 0; jt <= it; ++jt, ++item) {
          if ((item & 3) != wave) continue;
          const uint16_t* left = which == 0 ? sm.u.qk.k : sm.u.qk.q;
          f32x4 acc = {};
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(left + (16 * it + n16) * kQS + 32 * s + 8 * g4);
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(sm.u.qk.k + (16 * jt + n16) * kQS + 32 * s + 8 * g4);
            acc = mfma_bf16_16x16x32(av, bv, acc);
          }
          const int j = 16 * jt + n16;
          const float rkj = sm.rk[j], Gj = sm.G[j];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = 16 * it + 4 * g4 + r;
            const bool on = (sm.anc[i] >> j) & 1ull;
            if (which == 0) {
              sm.at[j * LDA + i] =
                  (on && j < i) ? sm.beta[i] * sm.rk[i] * rkj * acc[r] * __expf(sm.G[i] - Gj) : 0.f;
            } else {
              sm.pq[i * LDA + j] = on ? sm.rq[i] * rkj * acc[r] * __expf(sm.G[i] - Gj) : 0.f;
            }
          }
        }
  }

  // ---- 6. Cq = q_raw S0, Ck = k_raw S0 for the wave's 32 columns.  k-step s,
  // lane group g, element e -> k = 32s + 4g + e (e < 4), 32s + 16 + 4g + e-4.
  f32x4 cq[MT][2], ck[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      cq[mt][t] = f32x4{};
      ck[mt][t] = f32x4{};
    }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float x[8] = {s0r[t][2 * s][0],     s0r[t][2 * s][1],     s0r[t][2 * s][2],     s0r[t][2 * s][3],
                          s0r[t][2 * s + 1][0], s0r[t][2 * s + 1][1], s0r[t][2 * s + 1][2], s0r[t][2 * s + 1][3]};
      bf16x8 bhi, blo;
      split_bf16x8(x, bhi, blo);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int off = (16 * mt + n16) * kQS + 32 * s + 4 * g4;
        const bf16x8 aq = lds_bf16x8_split(sm.u.qk.q, off);
        const bf16x8 ak = lds_bf16x8_split(sm.u.qk.k, off);
        cq[mt][t] = mfma_bf16_16x16x32(aq, bhi, cq[mt][t]);
        ck[mt][t] = mfma_bf16_16x16x32(ak, bhi, ck[mt][t]);
        cq[mt][t] = mfma_bf16_16x16x32(aq, blo, cq[mt][t]);
        ck[mt][t] = mfma_bf16_16x16x32(ak, blo, ck[mt][t]);
      }
    }
  }
  __syncthreads();  // q/k reads done: the union now holds the transposed tiles

  // ---- 7. Ck to [column][node] in the wave's own slice
  float* ct = sm.u.ct[wave];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      *reinterpret_cast<f32x4*>(&ct[(16 * t + n16) * LDA + 16 * mt + 4 * g4]) = ck[mt][t];
      if constexpr (NP == 64)
        *reinterpret_cast<f32x4*>(&sm.cqs[wave * 32 * LDA + (16 * t + n16) * LDA + 16 * mt + 4 * g4]) = cq[mt][t];
    }
  __syncthreads();

  // ---- 8. (I + A) vn = diag(beta)(v - e^G rk Ck), lane = value column; both
  // halves of the wave solve the same column (no cross-lane traffic).
  const int c = lane & 31, hf = lane >> 5;
  const int vcol = 32 * wave + c;
  float x0[32], x1[32];  // nodes 0..31 and (NP = 64) 32..63
  auto rhs = [&](float (&x)[32], int base) {
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) {
      const int i = base + ii;
      const float vv = bf16_bits_to_f32(sm.v[i * kQS + vcol]);
      x[ii] = sm.beta[i] * (vv - sm.eG[i] * sm.rk[i] * ct[c * LDA + i]);
    }
  };
  rhs(x0, 0);
  if constexpr (NP == 64) rhs(x1, 32);
  solve_block32<LDA>(x0, sm.at, 0);
  materialize32(x0);
  if constexpr (NP == 64) {
    update_block32<LDA>(x1, x0, sm.at, 0, 32);
    solve_block32<LDA>(x1, sm.at, 32);
    materialize32(x1);
  }
  __syncthreads();  // every lane has read its Ck column
  auto save = [&](const float (&x)[32], int base) {
    if (hf == 0) {
#pragma unroll
      for (int i = 0; i < 32; i += 4)
        *reinterpret_cast<f32x4*>(&ct[c * LDA + base + i]) = f32x4{x[i], x[i + 1], x[i + 2], x[i + 3]};
    }
    if (p.aux_v) {
      float* dv = p.aux_v + (int64_t)h * p.aux_v_h_stride + row0 * p.aux_v_row_stride + vcol;
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        const int ii = base + i + hf;
        if (ii < n) dv[ii * p.aux_v_row_stride] = hf ? x[i + 1] : x[i];
      }
    }
  };
  save(x0, 0);
  if constexpr (NP == 64) save(x1, 32);
  __syncthreads();

  // ---- 9. o = e^G rq Cq + Pq vn in the 16x16 layout; Pq is lower triangular,
  // so row tile mt needs nodes m < 16(mt+1) only.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 cqv = cq[mt][t];
      if constexpr (NP == 64)
        cqv = *reinterpret_cast<const f32x4*>(&sm.cqs[wave * 32 * LDA + (16 * t + n16) * LDA + 16 * mt + 4 * g4]);
      f32x4 acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * mt + 4 * g4 + r;
        acc[r] = sm.eG[i] * sm.rq[i] * cqv[r];
      }
#pragma unroll
      for (int s = 0; s < 4 * (mt + 1); ++s) {
        const float a = sm.pq[(16 * mt + n16) * LDA + 4 * s + g4];
        const float bv = ct[(16 * t + n16) * LDA + 4 * s + g4];
        acc = mfma_f32_16x16x4(a, bv, acc);
      }
      const int col = 32 * wave + 16 * t + n16;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * mt + 4 * g4 + r;
        if (i < n) st_f(p.o, (row0 + i) * p.o_row_stride + (int64_t)h * p.o_h_stride + col, p.o_dtype, acc[r]);
      }
    }
}

int launch_tree_verify(const dft_verify_args* a, hipStream_t stream) {
  VerifyParams P;
  P.a = *a;
  const uintptr_t sp = reinterpret_cast<uintptr_t>(a->state);
  P.s0_vec = a->state_k_stride == 1 && (sp % 16) == 0 && (a->state_v_stride % 4) == 0 &&
             (a->state_h_stride % 4) == 0 && (a->state_slot_stride % 4) == 0;
  P.auxk_vec = a->aux_k && (reinterpret_cast<uintptr_t>(a->aux_k) % 16) == 0 && (a->aux_k_row_stride % 4) == 0 &&
               (a->aux_k_h_stride % 4) == 0;
  const dim3 grid((unsigned)(a->batch * a->hv)), block(256);
  if (a->n_nodes <= 32)
    hipLaunchKernelGGL(tree_verify_kernel<32>, grid, block, 0, stream, P);
  else
    hipLaunchKernelGGL(tree_verify_kernel<64>, grid, block, 0, stream, P);
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
