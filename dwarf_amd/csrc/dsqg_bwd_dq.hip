// DSQG backward, VALU path (fp32 and bf16).  Three launches, no global atomics
// (this file: launch 1; dsqg_bwd_dkdv.hip: launch 2; dsqg_bwd.hip: launch 3 and the driver):
//
//  1. bwd_dq_kernel (query-centric).  Per query row n: recompute s_j and alpha_j = exp(s_j - lse)
//     from the forward's lse, u_j = dOut.v_j, D' = sum_j alpha_j u_j (= dOut . o computed in
//     fp32 from the taps, never from the rounded output), dS_j = a alpha_j (u_j - D'), then
//     dq = c sum_j dS_j (g_j k_j + se_j).  D' goes to the workspace for launch 2.  The
//     parameter gradients (dbias, dse, dg, da) are summed over the workgroup's rows in a fixed
//     order and written as one partial per workgroup.
//  2. bwd_dkdv_kernel (key-centric).  Key row m gathers the queries n = m + delta_j that read
//     it: dv_m = sum_j a alpha_j(n) dOut_n,  dk_m = c sum_j g_j dS_j(n) q_n.  The queries of the
//     dense window, rows [m0, m0+QPB+W), are staged in LDS with their lse and D'.
//  3. bwd_reduce_kernel: sums the per-workgroup partials in a fixed order (deterministic).
//
// Follows _bwd_dq_v3 / _bwd_dkdv_v3 (kernels/dsqg_attention_v3.py:198-352), which use
// D = dO . out from the bf16 output (_compute_D_v3, :170-191) and global atomics for dpb/dse.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"

namespace dsqg {

template <typename T, int D, int JMAX, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void bwd_dq_kernel(BwdParams p) {
  constexpr int G = lanes_per_row(D);  // lanes with 8g >= D (D = 80, 96) hold zeros
  constexpr int QPB = kBlock / G;
  constexpr int ROWS = QPB + kMaxWindow;
  constexpr int CPR = D * (int)sizeof(T) / 16;
  constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int JS = JMAX + 1;              // padded row stride of the dS tables
  constexpr int SE_PER_T = (JMAX * D + kBlock - 1) / kBlock;

  __shared__ __align__(16) T sK[ROWS * D];
  __shared__ __align__(16) T sV[ROWS * D];
  __shared__ __align__(16) float sSE[HAS_SE ? JMAX * D : 1];
  __shared__ float sBias[JMAX];
  __shared__ float sGain[JMAX];
  __shared__ float sdS[QPB * JS];
  __shared__ float sdG[QPB * JS];
  __shared__ __align__(16) float sQ[QPB * D];
  __shared__ float sDp[QPB];

  const int tid = threadIdx.x;
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int bh = lb / p.n_chunks, chunk = lb - bh * p.n_chunks;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const float c = p.scale;
  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const bool se_grad = p.part_se != nullptr, g_grad = p.part_gain != nullptr;

  const T* qb = static_cast<const T*>(p.q) + b * p.qs.b + h * p.qs.h;
  const T* kb = static_cast<const T*>(p.k) + b * p.ks.b + h * p.ks.h;
  const T* vb = static_cast<const T*>(p.v) + b * p.vs.b + h * p.vs.h;
  const T* dob = static_cast<const T*>(p.dout) + b * p.dos.b + h * p.dos.h;
  T* dqb = static_cast<T*>(p.dq) + b * p.dqs.b + h * p.dqs.h;
  const long long rowbase = ((long long)b * p.H + h) * N;

  for (int j = tid; j < J; j += kBlock) {
    sBias[j] = p.pos_bias[j * p.H + h];
    sGain[j] = p.score_gain ? p.score_gain[h * J + j] : 1.0f;
  }
  if constexpr (HAS_SE) {
    for (int e = tid; e < J * D; e += kBlock) sSE[e] = p.scale_embed[e];
  }

  float acc_bias = 0.f, acc_gain = 0.f, acc_if = 0.f;
  float acc_se[SE_PER_T];
#pragma unroll
  for (int i = 0; i < SE_PER_T; ++i) acc_se[i] = 0.f;

  const int qi = tid / G, g = tid - qi * G;
  const int d0 = g * 8;
  const bool lane_ok = d0 < D;
  const int t_begin = chunk * p.tiles_per_block;
  const int t_end = min(p.n_tiles, t_begin + p.tiles_per_block);

  for (int tile = t_begin; tile < t_end; ++tile) {
    const int n0 = tile * QPB;
    const int base = n0 - W;
    __syncthreads();  // previous tile's LDS readers are done
    for (int ci = tid; ci < (QPB + W) * CPR; ci += kBlock) {
      const int r = ci / CPR, cc = ci - r * CPR;
      const int m = base + r;
      if (m >= 0 && m < N) {
        st16(sK + r * D + cc * EPC, ld16(kb + m * p.ks.n + cc * EPC));
        st16(sV + r * D + cc * EPC, ld16(vb + m * p.vs.n + cc * EPC));
      }
    }
    __syncthreads();

    const int n = n0 + qi;
    const bool row_ok = n < N;
    float q[8], dO[8];
    float lse = 0.f;
    if (row_ok) lse = p.lse[rowbase + n];
    if (row_ok && lane_ok) {
      Vec8<T>::load(qb + n * p.qs.n + d0, q);
      Vec8<T>::load(dob + n * p.dos.n + d0, dO);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { q[e] = 0.f; dO[e] = 0.f; }
    }

    float al[JMAX], u[JMAX], qk[JMAX];
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
      if (j < J) {
        const int m = n - p.taps.delta[j];
        const bool ok = row_ok && m >= 0;
        float ps = 0.f, pk = 0.f, pu = 0.f;
        if (ok && lane_ok) {
          float kx[8], vx[8];
          if (j <= W) {
            Vec8<T>::load(sK + (m - base) * D + d0, kx);
            Vec8<T>::load(sV + (m - base) * D + d0, vx);
          } else {
            Vec8<T>::load(kb + m * p.ks.n + d0, kx);
            Vec8<T>::load(vb + m * p.vs.n + d0, vx);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) { pk = fmaf(q[e], kx[e], pk); pu = fmaf(dO[e], vx[e], pu); }
          ps = pk * sGain[j];
          if constexpr (HAS_SE) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ps = fmaf(q[e], sSE[j * D + d0 + e], ps);
          }
        }
        const float ts = group_sum<G>(ps);
        const float tu = group_sum<G>(pu);
        qk[j] = g_grad ? c * group_sum<G>(pk) : 0.f;
        al[j] = ok ? __expf(fmaf(ts, c, sBias[j]) - lse) : 0.f;
        u[j] = tu;
      }
    }
    float Dp = 0.f;
#pragma unroll
    for (int j = 0; j < JMAX; ++j)
      if (j < J) Dp = fmaf(al[j], u[j], Dp);

    float dq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) dq[e] = 0.f;
#pragma unroll
    for (int j = 0; j < JMAX; ++j) {
      if (j < J) {
        const float dS = a * al[j] * (u[j] - Dp);
        u[j] = dS;
        if (al[j] > 0.f && lane_ok) {
          const int m = n - p.taps.delta[j];
          float kx[8];
          if (j <= W) Vec8<T>::load(sK + (m - base) * D + d0, kx);
          else Vec8<T>::load(kb + m * p.ks.n + d0, kx);
          const float dg = dS * sGain[j];
#pragma unroll
          for (int e = 0; e < 8; ++e) dq[e] = fmaf(dg, kx[e], dq[e]);
          if constexpr (HAS_SE) {
#pragma unroll
            for (int e = 0; e < 8; ++e) dq[e] = fmaf(dS, sSE[j * D + d0 + e], dq[e]);
          }
        }
      }
    }
    if (row_ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) dq[e] *= c;
      if (lane_ok) Vec8<T>::store(dqb + n * p.dqs.n + d0, dq);
      if (g == 0) p.dpre[rowbase + n] = Dp;
    }

    // Per-row contributions to the parameter gradients (zero for rows past N).
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < JMAX; ++j) {
        if (j < J) {
          sdS[qi * JS + j] = row_ok ? u[j] : 0.f;
          sdG[qi * JS + j] = row_ok ? u[j] * qk[j] : 0.f;
        }
      }
      sDp[qi] = row_ok ? Dp : 0.f;
    }
    if (se_grad && lane_ok) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sQ[qi * D + d0 + e] = q[e];
    }
    __syncthreads();
    if (tid < J) {
      float sb = 0.f, sg = 0.f;
      for (int i = 0; i < QPB; ++i) {
        sb += sdS[i * JS + tid];
        sg += sdG[i * JS + tid];
      }
      acc_bias += sb;
      acc_gain += sg;
    }
    if (tid == 0) {
      float sa = 0.f;
      for (int i = 0; i < QPB; ++i) sa += sDp[i];
      acc_if += sa;
    }
    if (se_grad) {
#pragma unroll
      for (int k2 = 0; k2 < SE_PER_T; ++k2) {
        const int e = tid + k2 * kBlock;
        if (e < J * D) {
          const int j = e / D, d = e - j * D;
          float ssum = 0.f;
          for (int i = 0; i < QPB; ++i) ssum = fmaf(sdS[i * JS + j], sQ[i * D + d], ssum);
          acc_se[k2] += c * ssum;
        }
      }
    }
  }

  if (tid < J) {
    p.part_bias[(long long)lb * J + tid] = acc_bias;
    if (p.part_gain) p.part_gain[(long long)lb * J + tid] = acc_gain;
  }
  if (tid == 0 && p.part_if) p.part_if[lb] = acc_if;
  if (se_grad) {
#pragma unroll
    for (int k2 = 0; k2 < SE_PER_T; ++k2) {
      const int e = tid + k2 * kBlock;
      if (e < J * D) p.part_se[(long long)lb * J * D + e] = acc_se[k2];
    }
  }
}


template <typename T, int D>
static hipError_t launch_bwd_dq_d(const BwdParams& p, unsigned nb, hipStream_t st) {
  if (p.scale_embed)
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kMaxTaps, true>), dim3(nb), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kMaxTaps, false>), dim3(nb), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_bwd_dq_dtype(const BwdParams& p, int D, unsigned nb, hipStream_t st) {
  switch (D) {
    case 32: return launch_bwd_dq_d<T, 32>(p, nb, st);
    case 64: return launch_bwd_dq_d<T, 64>(p, nb, st);
    case 80: return launch_bwd_dq_d<T, 80>(p, nb, st);
    case 96: return launch_bwd_dq_d<T, 96>(p, nb, st);
    case 128: return launch_bwd_dq_d<T, 128>(p, nb, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int D, unsigned nblocks, hipStream_t st) {
  if (bwd_mfma_supported(p, D, dtype)) return launch_bwd_dq_mfma(p, D, nblocks, st);
  return dtype == 0 ? launch_bwd_dq_dtype<float>(p, D, nblocks, st) : hipErrorNotSupported;
}

}  // namespace dsqg
