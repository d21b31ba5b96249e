// Fused GDN tree verify for gfx950: one workgroup (4 wave64) per
// (request, v-head) does prepare + (I+A)^-1 + finish of
// tree_kernels.py:135-208 in a single pass over the recurrent state.
//
// Math (per head; q_n, k_n normalised, rq/rk the row scales, so that
// q_n = rq * q_raw and k_n = rk * k_raw with q_raw/k_raw exact bf16):
//   G_i   = sum_{j anc-or-self i} g_j
//   A_ij  = [j strict anc i] beta_i (k_n,i . k_n,j) e^{G_i - G_j}
//   X     = (I + A)^-1
//   Cq    = q_raw S0,  Ck = k_raw S0                  (bf16 MFMA, S0 split hi+lo)
//   vn    = X diag(beta) (v - diag(e^G rk) Ck)        (= U - Wk S0 of :182-186)
//   o     = diag(e^G rq) Cq + (Pq) vn,  Pq_ij = [j anc-or-self i] (q_n,i . k_n,j) e^{G_i-G_j}
// The S0 contraction is the only part that touches the 64 KiB state; its
// left operand is the raw bf16 q/k rows, so only S0 needs the hi/lo split
// (two MFMAs per product, ~2^-17 relative).
//
// Layout of the work: wave w owns the 32 value columns [32w, 32w+32); each
// lane streams 64 contiguous fp32 of one state column (k-contiguous pool
// layout) straight into the MFMA B-operand registers, so the state is read
// once, coalesced, without an LDS round trip.  The 32x32 accumulators of
// Cq/Ck are consumed in place as B operands of the fp32 MFMAs of phase 3.
#include "dft_device.h"

namespace dft {

constexpr int kD = 128;
constexpr int kQS = kD + 8;  // LDS row stride (bf16) of q/k rows: 272 B

struct VerifyParams {
  dft_verify_args a;
  int s0_vec;  // state rows 16-byte aligned with k stride 1
};

template <int NP>
struct VerifySmem {
  uint16_t q[NP * kQS];
  uint16_t k[NP * kQS];
  float ax[NP * (NP + 1)];  // A, then X = (I+A)^-1 in place
  float pq[NP * (NP + 1)];
  float g[NP], G[NP], beta[NP], rq[NP], rk[NP];
  uint64_t anc[NP];
};

// Forward substitution by one wave: lane j keeps column j of X in registers.
// X[i][j] = delta_ij - sum_{m<i} A[i][m] X[m][j].
template <int NP>
__device__ __forceinline__ void invert_unit_lower(float* ax, int lane) {
  constexpr int LD = NP + 1;
  const int j = lane;
  float x[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float s0 = (i == j) ? 1.f : 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
    for (int m = 0; m < i; ++m) {
      const float a = ax[i * LD + m];
      if ((m & 3) == 0) s0 -= a * x[m];
      else if ((m & 3) == 1) s1 -= a * x[m];
      else if ((m & 3) == 2) s2 -= a * x[m];
      else s3 -= a * x[m];
    }
    x[i] = (s0 + s1) + (s2 + s3);
  }
  // every read of A above has been consumed, so X can overwrite it
  if (j < NP) {
#pragma unroll
    for (int i = 0; i < NP; ++i) ax[i * LD + j] = (i >= j) ? x[i] : 0.f;
  }
}

template <int NP>
__global__ void __launch_bounds__(256) tree_verify_kernel(const VerifyParams P) {
  constexpr int MT = NP / 32;
  constexpr int LD = NP + 1;
  const dft_verify_args& p = P.a;
  __shared__ VerifySmem<NP> sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, half = lane >> 5;

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

  // ---- 1. state tile loads first: lane (wave w, l32, half) holds
  // S0[k = 64*half + e][v = 32w + l32] for e < 64.
  const int vcol = 32 * wave + l32;
  float s0r[64];
  if (P.s0_vec) {
    const f32x4* src = reinterpret_cast<const f32x4*>(S0 + vcol * p.state_v_stride + 64 * half);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const f32x4 t = __builtin_nontemporal_load(src + i);
      s0r[4 * i + 0] = t.x;
      s0r[4 * i + 1] = t.y;
      s0r[4 * i + 2] = t.z;
      s0r[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 64; ++e)
      s0r[e] = S0[vcol * p.state_v_stride + (int64_t)(64 * half + e) * p.state_k_stride];
  }

  const int KD = p.hk * kD;
  const int64_t ys = p.y_row_stride;
  const uint16_t* ybase = reinterpret_cast<const uint16_t*>(p.y) + row0 * ys;

  // ---- 2. v values in the accumulator layout used by phase 3
  float vr[MT][16];
  {
    const uint16_t* yv = ybase + 2 * KD + h * kD + vcol;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = 32 * mt + acc_row(r, half);
        vr[mt][r] = i < n ? bf16_bits_to_f32(yv[i * ys]) : 0.f;
      }
  }

  // ---- 3. raw q/k rows to LDS, gates, ancestry
  {
    const uint16_t* yq = ybase + hk * kD;
    const uint16_t* yk = yq + KD;
    for (int c = tid; c < NP * 16; c += 256) {
      const int i = c >> 4, ch = (c & 15) * 8;
      uint4 vq = {0u, 0u, 0u, 0u}, vk = {0u, 0u, 0u, 0u};
      if (i < n) {
        vq = *reinterpret_cast<const uint4*>(yq + i * ys + ch);
        vk = *reinterpret_cast<const uint4*>(yk + i * ys + ch);
      }
      *reinterpret_cast<uint4*>(&sm.q[i * kQS + ch]) = vq;
      *reinterpret_cast<uint4*>(&sm.k[i * kQS + ch]) = vk;
    }
  }
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
    const uint16_t* rowp = (tid < NP ? sm.q : sm.k) + (tid % NP) * kQS;
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
    uint64_t bits = sm.anc[i];
    float G = 0.f;
    while (bits) {
      const int j = __builtin_ctzll(bits);
      G += sm.g[j];
      bits &= bits - 1;
    }
    sm.G[i] = G;
  }
  __syncthreads();

  // ---- 5. Gram tiles: wave 0 builds A from k k^T, wave 1 builds Pq from q k^T
  if (wave < 2) {
    const uint16_t* left = wave == 0 ? sm.k : sm.q;
#pragma unroll
    for (int rt = 0; rt < MT; ++rt)
#pragma unroll
      for (int ct = 0; ct <= rt; ++ct) {
        f32x16 acc = {};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const bf16x8 av = *reinterpret_cast<const bf16x8*>(left + (32 * rt + l32) * kQS + 16 * s + 8 * half);
          const bf16x8 bv = *reinterpret_cast<const bf16x8*>(sm.k + (32 * ct + l32) * kQS + 16 * s + 8 * half);
          acc = mfma_bf16_32x32x16(av, bv, acc);
        }
        const int j = 32 * ct + l32;
        const float rkj = sm.rk[j], Gj = sm.G[j];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = 32 * rt + acc_row(r, half);
          const bool on = (sm.anc[i] >> j) & 1ull;
          if (wave == 0) {
            const float val = (on && j < i) ? sm.beta[i] * sm.rk[i] * rkj * acc[r] * __expf(sm.G[i] - Gj) : 0.f;
            sm.ax[i * LD + j] = val;
          } else {
            const float val = on ? sm.rq[i] * rkj * acc[r] * __expf(sm.G[i] - Gj) : 0.f;
            sm.pq[i * LD + j] = val;
          }
        }
      }
  }
  __syncthreads();

  // ---- 6. X = (I+A)^-1 on wave 0; meanwhile every wave contracts its
  // state columns: Cq = q_raw S0, Ck = k_raw S0 (k index of lane group
  // `half` at step s: 64*half + 8*s + e, identical for both operands).
  if (wave == 0) invert_unit_lower<NP>(sm.ax, lane);

  f32x16 accq[MT], acck[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    accq[mt] = f32x16{};
    acck[mt] = f32x16{};
  }
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    bf16x8 bhi, blo;
    split_bf16x8(&s0r[8 * s], bhi, blo);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int off = (32 * mt + l32) * kQS + 64 * half + 8 * s;
      const bf16x8 aq = *reinterpret_cast<const bf16x8*>(sm.q + off);
      const bf16x8 ak = *reinterpret_cast<const bf16x8*>(sm.k + off);
      accq[mt] = mfma_bf16_32x32x16(aq, bhi, accq[mt]);
      acck[mt] = mfma_bf16_32x32x16(ak, bhi, acck[mt]);
      accq[mt] = mfma_bf16_32x32x16(aq, blo, accq[mt]);
      acck[mt] = mfma_bf16_32x32x16(ak, blo, acck[mt]);
    }
  }
  __syncthreads();  // X visible to every wave

  // ---- 7. phase 3: vn = X diag(beta)(v - e^G rk Ck);  o = e^G rq Cq + Pq vn
  float wb[MT][16];
  f32x16 oacc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * mt + acc_row(r, half);
      const float eG = __expf(sm.G[i]);
      wb[mt][r] = sm.beta[i] * (vr[mt][r] - eG * sm.rk[i] * acck[mt][r]);
      oacc[mt][r] = eG * sm.rq[i] * accq[mt][r];
    }

  f32x16 vn[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    vn[mt] = f32x16{};
#pragma unroll
    for (int kt = 0; kt <= mt; ++kt)
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const float a = sm.ax[(32 * mt + l32) * LD + 32 * kt + acc_row(s, half)];
        vn[mt] = mfma_f32_32x32x2(a, wb[kt][s], vn[mt]);
      }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int kt = 0; kt <= mt; ++kt)
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const float a = sm.pq[(32 * mt + l32) * LD + 32 * kt + acc_row(s, half)];
        oacc[mt] = mfma_f32_32x32x2(a, vn[kt][s], oacc[mt]);
      }

  // ---- 8. stores
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = 32 * mt + acc_row(r, half);
      if (i < n) {
        st_f(p.o, (row0 + i) * p.o_row_stride + (int64_t)h * p.o_h_stride + vcol, p.o_dtype, oacc[mt][r]);
        if (p.aux_v) p.aux_v[(int64_t)h * p.aux_v_h_stride + (row0 + i) * p.aux_v_row_stride + vcol] = vn[mt][r];
      }
    }
  const bool per_khead = (p.flags & DFT_VERIFY_AUX_K_PER_KHEAD) != 0;
  if (p.aux_k && (!per_khead || rr == 0)) {
    float* dk = p.aux_k + (int64_t)(per_khead ? hk : h) * p.aux_k_h_stride + row0 * p.aux_k_row_stride;
    for (int c = tid; c < n * kD; c += 256) {
      const int i = c >> 7, d = c & (kD - 1);
      dk[i * p.aux_k_row_stride + d] = bf16_bits_to_f32(sm.k[i * kQS + d]) * sm.rk[i];
    }
  }
  if (p.aux_g && tid < n) p.aux_g[(int64_t)h * p.aux_g_h_stride + (row0 + tid) * p.aux_g_row_stride] = sm.G[tid];
}

int launch_tree_verify(const dft_verify_args* a, hipStream_t stream) {
  VerifyParams P;
  P.a = *a;
  const uintptr_t sp = reinterpret_cast<uintptr_t>(a->state);
  P.s0_vec = a->state_k_stride == 1 && (sp % 16) == 0 && (a->state_v_stride % 4) == 0 &&
             (a->state_h_stride % 4) == 0 && (a->state_slot_stride % 4) == 0;
  const dim3 grid((unsigned)(a->batch * a->hv)), block(256);
  if (a->n_nodes <= 32)
    hipLaunchKernelGGL(tree_verify_kernel<32>, grid, block, 0, stream, P);
  else
    hipLaunchKernelGGL(tree_verify_kernel<64>, grid, block, 0, stream, P);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

// ---------------------------------------------------------------------------
// standalone in-place (I+A)^-1, one wave per matrix (fc1_block_inverse.py)
// ---------------------------------------------------------------------------
template <int NP>
__global__ void __launch_bounds__(64) block_inverse_kernel(float* x, int n, int64_t mat_stride) {
  constexpr int LD = NP + 1;
  __shared__ float ax[NP * LD];
  float* m = x + (int64_t)blockIdx.x * mat_stride;
  const int lane = threadIdx.x;
  if (lane < NP)
    for (int i = 0; i < NP; ++i)  // strict lower part of row i; padding is zero
      ax[i * LD + lane] = (i < n && lane < i) ? m[i * n + lane] : 0.f;
  __syncthreads();
  invert_unit_lower<NP>(ax, lane);
  __syncthreads();
  for (int i = 0; i < n; ++i)
    if (lane < n) m[i * n + lane] = ax[i * LD + lane];
}

int launch_block_inverse(float* x, int n_mats, int n, int64_t mat_stride, hipStream_t stream) {
  if (n <= 32)
    hipLaunchKernelGGL(block_inverse_kernel<32>, dim3(n_mats), dim3(64), 0, stream, x, n, mat_stride);
  else
    hipLaunchKernelGGL(block_inverse_kernel<64>, dim3(n_mats), dim3(64), 0, stream, x, n, mat_stride);
  return hipGetLastError() == hipSuccess ? DFT_OK : DFT_ERR_LAUNCH;
}

}  // namespace dft
