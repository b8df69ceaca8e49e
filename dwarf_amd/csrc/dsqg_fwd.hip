// DSQG forward, VALU path: fp32, and bf16 offset tables outside the MFMA kernel's reach
// (more than kMaxSparse taps beyond the dense window).
//
// One workgroup = one (b,h) and a tile of QPB query rows.  Each query row is owned by a group
// of G consecutive lanes (D/8 rounded up to a power of two), lane g holding elements
// [8g, 8g+8) of the row (lanes with 8g >= D hold zeros), so one row is one coalesced
// D*sizeof(T)-byte access by the group.  The dense window (delta = 0..W) of K and
// V for the tile, rows [n0-W, n0+QPB), is staged in LDS once and reused by every row of the
// tile; the long-range taps are gathered straight from global memory (the rows of tap delta
// for the tile are the contiguous block [n0-delta, n0-delta+QPB)).  Scores are kept in
// registers (JMAX of them per row), so the softmax is a plain two-pass max/exp/sum with no
// rescaling of the accumulator.
//
// Semantics follow _fwd_v3 (kernels/dsqg_attention_v3.py:60-163): s_j = c q.k_j + b[j,h]
// + c q.se_j (here with the optional g[h,j] on the content term), taps with n - delta_j < 0
// masked out of the softmax, out = sum_j alpha_j v_j (times the optional a[h]), lse = m + log l.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"

namespace dsqg {

template <typename T, int D, int JMAX, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void fwd_valu_kernel(FwdParams p) {
  constexpr int G = lanes_per_row(D);
  constexpr int QPB = kBlock / G;
  constexpr int ROWS = QPB + kMaxWindow;
  constexpr int CPR = D * (int)sizeof(T) / 16;  // 16-byte chunks per row

  __shared__ __align__(16) T sK[ROWS * D];
  __shared__ __align__(16) T sV[ROWS * D];
  __shared__ __align__(16) float sSE[HAS_SE ? JMAX * D : 1];
  __shared__ float sBias[JMAX];
  __shared__ float sGain[JMAX];

  const int tid = threadIdx.x;
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int bh = lb / p.n_tiles, tile = lb - bh * p.n_tiles;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const int n0 = tile * QPB;
  const int base = n0 - W;  // first staged row

  const T* qb = static_cast<const T*>(p.q) + b * p.qs.b + h * p.qs.h;
  const T* kb = static_cast<const T*>(p.k) + b * p.ks.b + h * p.ks.h;
  const T* vb = static_cast<const T*>(p.v) + b * p.vs.b + h * p.vs.h;

  // Stage K/V rows [base, n0+QPB) that exist.
  const int nrows = QPB + W;
  for (int c = tid; c < nrows * CPR; c += kBlock) {
    const int r = c / CPR, cc = c - r * CPR;
    const int m = base + r;
    if (m >= 0 && m < N) {
      st16(sK + r * D + cc * (16 / sizeof(T)), ld16(kb + m * p.ks.n + cc * (16 / sizeof(T))));
      st16(sV + r * D + cc * (16 / sizeof(T)), ld16(vb + m * p.vs.n + cc * (16 / sizeof(T))));
    }
  }
  for (int j = tid; j < J; j += kBlock) {
    sBias[j] = p.pos_bias[j * p.H + h];
    sGain[j] = p.score_gain ? p.score_gain[h * J + j] : 1.0f;
  }
  if constexpr (HAS_SE) {
    for (int e = tid; e < J * D; e += kBlock) sSE[e] = p.scale_embed[e];
  }
  __syncthreads();

  const int qi = tid / G, g = tid - qi * G;
  const int n = n0 + qi;
  const bool row_ok = n < N;
  const int d0 = g * 8;
  const bool lane_ok = d0 < D;  // lanes past the row (D = 80, 96) hold zeros
  const float c = p.scale;

  float q[8];
  if (row_ok && lane_ok) {
    Vec8<T>::load(qb + n * p.qs.n + d0, q);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = 0.f;
  }

  float s[JMAX];
#pragma unroll
  for (int j = 0; j < JMAX; ++j) {
    if (j < J) {
      const int dl = p.taps.delta[j];
      const int m = n - dl;
      const bool ok = row_ok && m >= 0;
      float part = 0.f;
      if (ok && lane_ok) {
        float kx[8];
        if (j <= W) Vec8<T>::load(sK + (m - base) * D + d0, kx);
        else Vec8<T>::load(kb + m * p.ks.n + d0, kx);
        float pk = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) pk = fmaf(q[e], kx[e], pk);
        part = pk * sGain[j];
        if constexpr (HAS_SE) {
#pragma unroll
          for (int e = 0; e < 8; ++e) part = fmaf(q[e], sSE[j * D + d0 + e], part);
        }
      }
      const float tot = group_sum<G>(part);
      s[j] = ok ? fmaf(tot, c, sBias[j]) : -INFINITY;
    }
  }

  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < JMAX; ++j)
    if (j < J) mx = fmaxf(mx, s[j]);
  if (!row_ok) mx = 0.f;

  float l = 0.f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int j = 0; j < JMAX; ++j) {
    if (j < J) {
      const float pj = __expf(s[j] - mx);
      l += pj;
      if (pj > 0.f && lane_ok) {
        const int m = n - p.taps.delta[j];
        float vx[8];
        if (j <= W) Vec8<T>::load(sV + (m - base) * D + d0, vx);
        else Vec8<T>::load(vb + m * p.vs.n + d0, vx);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(pj, vx[e], acc[e]);
      }
    }
  }

  if (row_ok) {
    const float a = p.if_gain ? p.if_gain[h] : 1.0f;
    const float inv = a / l;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = acc[e] * inv;
    T* ob = static_cast<T*>(p.out) + b * p.os.b + h * p.os.h + n * p.os.n + d0;
    if (lane_ok) Vec8<T>::store(ob, o);
    if (p.lse && g == 0) p.lse[((long long)b * p.H + h) * N + n] = mx + __logf(l);
  }
}

template <typename T, int D, int JMAX>
static hipError_t launch_fwd_t(const FwdParams& p0, hipStream_t st) {
  FwdParams p = p0;
  constexpr int QPB = kBlock / lanes_per_row(D);
  p.n_tiles = (p.N + QPB - 1) / QPB;
  const long long nblocks = (long long)p.B * p.H * p.n_tiles;
  if (nblocks == 0) return hipSuccess;
  if (p.scale_embed)
    hipLaunchKernelGGL((fwd_valu_kernel<T, D, JMAX, true>), dim3((unsigned)nblocks), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL((fwd_valu_kernel<T, D, JMAX, false>), dim3((unsigned)nblocks), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_fwd_d(const FwdParams& p, hipStream_t st) {
  return launch_fwd_t<T, D, kMaxTaps>(p, st);
}

template <typename T>
static hipError_t launch_fwd_dtype(const FwdParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return launch_fwd_d<T, 32>(p, st);
    case 64: return launch_fwd_d<T, 64>(p, st);
    case 80: return launch_fwd_d<T, 80>(p, st);
    case 96: return launch_fwd_d<T, 96>(p, st);
    case 128: return launch_fwd_d<T, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_fwd(const FwdParams& p, int dtype, int D, hipStream_t st) {
  // fp32 runs these VALU kernels; bf16 runs only the MFMA kernel (the ABI rejects a bf16 call
  // it cannot take with DSQG_EUNSUPPORTED before getting here).
  if (dtype == 0) return launch_fwd_dtype<float>(p, D, st);
  if (fwd_mfma_supported(p, D)) return launch_fwd_mfma(p, D, st);
  return hipErrorNotSupported;
}

}  // namespace dsqg
