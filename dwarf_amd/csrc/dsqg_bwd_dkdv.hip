// DSQG backward, launch 2: key-centric dk/dv (VALU path, fp32 and bf16).
//
// Key row m gathers the queries n = m + delta_j that read it:
//   dv_m = sum_j a alpha_j(n) dOut_n,   dk_m = c sum_j g_j dS_j(n) q_n,
// with alpha_j(n) = exp(s_j(n) - lse_n) and dS_j(n) = a alpha_j(n) (dOut_n.v_m - D'_n), D'_n
// written by launch 1.  The query rows of the dense window, [m0, m0+QPB+W), are staged in LDS
// with their lse and D'; long-range taps read the query rows [m0+delta, m0+delta+QPB) directly.
// Follows _bwd_dkdv_v3 (kernels/dsqg_attention_v3.py:282-352), which also needs no atomics.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_reduce.hpp"

namespace dsqg {

template <typename T, int D, int JMAX, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void bwd_dkdv_kernel(BwdParams p) {
  constexpr int G = lanes_per_row(D);  // lanes with 8g >= D (D = 80, 96) hold zeros
  constexpr int QPB = kBlock / G;
  constexpr int ROWS = QPB + kMaxWindow;
  constexpr int CPR = D * (int)sizeof(T) / 16;
  constexpr int EPC = 16 / (int)sizeof(T);

  __shared__ __align__(16) T sQ[ROWS * D];
  __shared__ __align__(16) T sDO[ROWS * D];
  __shared__ float sL[ROWS];
  __shared__ float sDp[ROWS];
  __shared__ __align__(16) float sSE[HAS_SE ? JMAX * D : 1];
  __shared__ float sBias[JMAX];
  __shared__ float sGain[JMAX];

  const int tid = threadIdx.x;
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int bh = lb / p.n_tiles_kv, tile = lb - bh * p.n_tiles_kv;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const float c = p.scale;
  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const int m0 = tile * QPB;

  const T* qb = static_cast<const T*>(p.q) + b * p.qs.b + h * p.qs.h;
  const T* kb = static_cast<const T*>(p.k) + b * p.ks.b + h * p.ks.h;
  const T* vb = static_cast<const T*>(p.v) + b * p.vs.b + h * p.vs.h;
  const T* dob = static_cast<const T*>(p.dout) + b * p.dos.b + h * p.dos.h;
  const long long rowbase = ((long long)b * p.H + h) * N;

  // Stage query-side rows [m0, m0+QPB+W) that exist.
  const int nrows = QPB + W;
  for (int ci = tid; ci < nrows * CPR; ci += kBlock) {
    const int r = ci / CPR, cc = ci - r * CPR;
    const int n = m0 + r;
    if (n < N) {
      st16(sQ + r * D + cc * EPC, ld16(qb + n * p.qs.n + cc * EPC));
      st16(sDO + r * D + cc * EPC, ld16(dob + n * p.dos.n + cc * EPC));
    }
  }
  for (int r = tid; r < nrows; r += kBlock) {
    const int n = m0 + r;
    if (n < N) { sL[r] = p.lse[rowbase + n]; sDp[r] = p.dpre[rowbase + n]; }
  }
  for (int j = tid; j < J; j += kBlock) {
    sBias[j] = p.pos_bias[j * p.H + h];
    sGain[j] = p.score_gain ? p.score_gain[h * J + j] : 1.0f;
  }
  if constexpr (HAS_SE) {
    for (int e = tid; e < J * D; e += kBlock) sSE[e] = p.scale_embed[e];
  }
  __syncthreads();

  const int ki = tid / G, g = tid - ki * G;
  const int m = m0 + ki;
  const bool key_ok = m < N;
  const int d0 = g * 8;
  const bool lane_ok = d0 < D;

  float kx[8], vx[8];
  if (key_ok && lane_ok) {
    Vec8<T>::load(kb + m * p.ks.n + d0, kx);
    Vec8<T>::load(vb + m * p.vs.n + d0, vx);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) { kx[e] = 0.f; vx[e] = 0.f; }
  }
  float dk[8], dv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { dk[e] = 0.f; dv[e] = 0.f; }

#pragma unroll
  for (int j = 0; j < JMAX; ++j) {
    if (j < J) {
      const int n = m + p.taps.delta[j];
      const bool ok = key_ok && n < N;
      float qx[8], dx[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) { qx[e] = 0.f; dx[e] = 0.f; }
      float ps = 0.f, pu = 0.f, lse = 0.f, Dp = 0.f;
      if (ok) {
        if (j <= W) {
          if (lane_ok) {
            Vec8<T>::load(sQ + (n - m0) * D + d0, qx);
            Vec8<T>::load(sDO + (n - m0) * D + d0, dx);
          }
          lse = sL[n - m0];
          Dp = sDp[n - m0];
        } else {
          if (lane_ok) {
            Vec8<T>::load(qb + n * p.qs.n + d0, qx);
            Vec8<T>::load(dob + n * p.dos.n + d0, dx);
          }
          lse = p.lse[rowbase + n];
          Dp = p.dpre[rowbase + n];
        }
        float pk = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) { pk = fmaf(qx[e], kx[e], pk); pu = fmaf(dx[e], vx[e], pu); }
        ps = pk * sGain[j];
        if constexpr (HAS_SE) {
          if (lane_ok) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ps = fmaf(qx[e], sSE[j * D + d0 + e], ps);
          }
        }
      }
      const float ts = group_sum<G>(ps);
      const float tu = group_sum<G>(pu);
      if (ok) {
        const float al = __expf(fmaf(ts, c, sBias[j]) - lse);
        const float dS = a * al * (tu - Dp);
        const float wv = a * al, wk = c * sGain[j] * dS;
#pragma unroll
        for (int e = 0; e < 8; ++e) { dv[e] = fmaf(wv, dx[e], dv[e]); dk[e] = fmaf(wk, qx[e], dk[e]); }
      }
    }
  }
  if (key_ok && lane_ok) {
    Vec8<T>::store(static_cast<T*>(p.dk) + b * p.dks.b + h * p.dks.h + m * p.dks.n + d0, dk);
    Vec8<T>::store(static_cast<T*>(p.dv) + b * p.dvs.b + h * p.dvs.h + m * p.dvs.n + d0, dv);
  }
}


template <typename T, int D>
static hipError_t launch_bwd_dkdv_d(const BwdParams& p, unsigned nb, hipStream_t st) {
  if (p.scale_embed)
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, D, kMaxTaps, true>), dim3(nb), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL((bwd_dkdv_kernel<T, D, kMaxTaps, false>), dim3(nb), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_bwd_dkdv_dtype(const BwdParams& p, int D, unsigned nb, hipStream_t st) {
  switch (D) {
    case 32: return launch_bwd_dkdv_d<T, 32>(p, nb, st);
    case 64: return launch_bwd_dkdv_d<T, 64>(p, nb, st);
    case 80: return launch_bwd_dkdv_d<T, 80>(p, nb, st);
    case 96: return launch_bwd_dkdv_d<T, 96>(p, nb, st);
    case 128: return launch_bwd_dkdv_d<T, 128>(p, nb, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int D, unsigned nblocks, hipStream_t st) {
  if (bwd_mfma_supported(p, D, dtype)) return launch_bwd_dkdv_mfma(p, D, nblocks, st);
  return dtype == 0 ? launch_bwd_dkdv_dtype<float>(p, D, nblocks, st) : hipErrorNotSupported;
}

hipError_t launch_bwd_dkdv_params(const BwdParams& p, const ReduceParams& r, int dtype, int D,
                                  unsigned nblocks, hipStream_t st) {
  if (bwd_mfma_supported(p, D, dtype)) {
    BwdParams pr = p;
    pr.red = r;
    pr.red_blocks = (int)((reduce_params_waves(r) + kBlock / 64 - 1) / (kBlock / 64));
    return launch_bwd_dkdv_mfma(pr, D, nblocks + (unsigned)pr.red_blocks, st);
  }
  const hipError_t e = launch_bwd_dkdv(p, dtype, D, nblocks, st);
  return e != hipSuccess ? e : launch_bwd_reduce_final(r, st);
}

}  // namespace dsqg
