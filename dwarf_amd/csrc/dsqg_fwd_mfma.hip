// DSQG forward, bf16 MFMA path (gfx950).
//
// Workgroup = one (b,h) and 64 query rows [n0, n0+64); wave w owns rows n0+16w .. +15.
//  1. The dense window, K/V rows [n0-32, n0+64), is copied once into LDS (zero rows outside
//     [0,N)).  Each wave's queries see the 48-key band [n0w-32, n0w+16) of it.
//  2. Scores for the band: S^T = K_band Q^T with v_mfma_f32_16x16x32_bf16 (A = key rows from
//     LDS, B = the wave's query rows, straight from global memory).  Lane l then holds query
//     column i = l%16 and keys 4*(l/16) + r of each 16-key block, i.e. delta = n - m is known
//     per register; taps outside delta in [0, W] (or before row 0) become -inf.
//  3. Long-range taps: for tap delta the key rows are the contiguous block n0w - delta + 0..15;
//     S^T_t = K_t Q^T is one 16x16 tile whose diagonal holds the 16 wanted scores (lane
//     16*(i/4) + i, register i%4).  The K rows are coalesced 16-byte loads from L2.
//  4. Optional q.se_j term: SE Q^T with the same MFMA, kept per wave in an LDS table
//     T[i][j] = bias[j] + c q_i . se_j; without scale_embed T is the bias row.
//  5. Softmax over each query's J taps in registers: the four lanes of a query column combine
//     max and sum with two cross-lane steps; lse = max + log(sum); the weights are normalised
//     (and scaled by the IF gain) before P V.
//  6. P V: O^T = V^T P^T with v_mfma_f32_16x16x16_bf16.  V^T comes from the row-major LDS tile
//     through ds_read_tr16_b64; P^T is already in B layout.  Long-range taps stage their V
//     rows [n0-delta, n0-delta+64) in a double-buffered LDS block and multiply by a diagonal
//     P^T that is non-zero in one register of the diagonal lane only.
//
// Semantics: _fwd_v3, kernels/dsqg_attention_v3.py:60-163 (plus score gain and IF gain).
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_mfma.hpp"

namespace dsqg {

// Loads this thread's 16-byte chunks of the 64-row block starting at row r0 (zero outside
// [0, N)) into registers; chunk c of the block is row c / CPR, column chunk c % CPR.
template <int CH, int CPR>
__device__ __forceinline__ void stage_rows(uint4 (&stg)[CH], const bf16_t* base, long long rs,
                                           int r0, int N, int tid) {
#pragma unroll
  for (int cI = 0; cI < CH; ++cI) {
    const int chunk = tid + cI * kBlock;
    const int r = chunk / CPR, cc = chunk - r * CPR;
    const int m = r0 + r;
    stg[cI] = (m >= 0 && m < N) ? ld16(base + m * rs + cc * 8) : zero16();
  }
}

template <int D, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void fwd_mfma_kernel(FwdParams p) {
  constexpr int QT = 64;                 // query rows per workgroup
  constexpr int KS = D / 32;             // 16x16x32 steps over the head dim
  constexpr int DB = D / 16;             // 16-wide head-dim blocks of the output
  constexpr int RK = D + 8;              // LDS row stride of K (16-byte natural reads)
  constexpr int RV = D + 16;             // LDS row stride of V (transposing reads)
  constexpr int WIN = QT + kMaxWindow;   // staged dense-window rows
  constexpr int CPR = D / 8;             // 16-byte chunks per row
  constexpr int CH = QT * CPR / kBlock;  // chunks per thread when staging a 64-row block
  constexpr int TS = 49;                 // row stride of the per-wave T table

  __shared__ __align__(16) bf16_t sK[WIN * RK];
  __shared__ __align__(16) bf16_t sV[WIN * RV];
  __shared__ __align__(16) bf16_t sVs[2][QT * RV];
  __shared__ __align__(16) bf16_t sSE[HAS_SE ? 48 * RK : 8];
  __shared__ float sT[HAS_SE ? 4 * 16 * TS : 1];
  __shared__ float sBias[kMaxTaps];
  __shared__ float sGain[kMaxTaps];

  const int tid = threadIdx.x;
  const int lb = xcd_logical_block(blockIdx.x, gridDim.x);
  const int bh = lb / p.n_tiles, tile = lb - bh * p.n_tiles;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const int NS = J - W - 1;
  const int n0 = tile * QT;
  const float c = p.scale;

  const bf16_t* qb = static_cast<const bf16_t*>(p.q) + b * p.qs.b + h * p.qs.h;
  const bf16_t* kb = static_cast<const bf16_t*>(p.k) + b * p.ks.b + h * p.ks.h;
  const bf16_t* vb = static_cast<const bf16_t*>(p.v) + b * p.vs.b + h * p.vs.h;

  for (int ci = tid; ci < WIN * CPR; ci += kBlock) {
    const int r = ci / CPR, cc = ci - r * CPR;
    const int m = n0 - kMaxWindow + r;
    const bool ok = m >= 0 && m < N;
    st16(sK + r * RK + cc * 8, ok ? ld16(kb + m * p.ks.n + cc * 8) : zero16());
    st16(sV + r * RV + cc * 8, ok ? ld16(vb + m * p.vs.n + cc * 8) : zero16());
  }
  for (int j = tid; j < J; j += kBlock) {
    sBias[j] = p.pos_bias[j * p.H + h];
    sGain[j] = p.score_gain ? p.score_gain[h * J + j] : 1.0f;
  }
  if constexpr (HAS_SE) {
    for (int e = tid; e < 48 * D; e += kBlock) {
      const int j = e / D, d = e - j * D;
      const __bf16 x = (__bf16)(j < J ? p.scale_embed[j * D + d] : 0.f);
      sSE[j * RK + d] = __builtin_bit_cast(bf16_t, x);
    }
  }
  __syncthreads();

  const int w = tid >> 6, l = tid & 63, i = l & 15, g = l >> 4;
  const int n0w = n0 + 16 * w;
  const int n = n0w + i;  // query row of this lane's MFMA column
  const bool row_ok = n < N;

  bf16x8_t qB[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qB[s] = as_bf16x8(row_ok ? ld16(qb + n * p.qs.n + 32 * s + 8 * g) : zero16());

  // Dense band scores.
  f32x4_t accS[3];
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    accS[kk] = zero4();
    const bf16_t* kr = sK + (16 * w + 16 * kk + i) * RK + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      accS[kk] = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(kr + 32 * s)), qB[s], accS[kk]);
  }

  float* sTw = sT + (HAS_SE ? w * 16 * TS : 0);
  if constexpr (HAS_SE) {
#pragma unroll
    for (int jb = 0; jb < 3; ++jb) {
      f32x4_t acc = zero4();
      const bf16_t* sr = sSE + (16 * jb + i) * RK + 8 * g;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(sr + 32 * s)), qB[s], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * jb + 4 * g + r;
        if (j < J) sTw[i * TS + j] = fmaf(c, acc[r], sBias[j]);
      }
    }
    __syncthreads();
  }

  float sd[12];
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dl = 32 - 16 * kk - 4 * g - r + i;  // n - m for key m of this register
      const bool ok = row_ok && dl >= 0 && dl <= W && n - dl >= 0;
      const int j = ok ? dl : 0;
      sd[kk * 4 + r] = ok ? fmaf(c * sGain[j], accS[kk][r], HAS_SE ? sTw[i * TS + j] : sBias[j]) : -INFINITY;
    }
  }

  const bool diag = g == (i >> 2);
  float ss[kMaxSparse];
#pragma unroll
  for (int t = 0; t < kMaxSparse; ++t) {
    ss[t] = -INFINITY;
    if (t < NS) {
      const int j = W + 1 + t;
      const int dl = p.taps.delta[j];
      const int mrow = n0w + i - dl;  // key row feeding A row i
      const bool in = mrow >= 0 && mrow < N;
      f32x4_t acc = zero4();
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = mfma_16x16x32(as_bf16x8(in ? ld16(kb + mrow * p.ks.n + 32 * s + 8 * g) : zero16()), qB[s], acc);
      const float raw = pick4(acc, i & 3);
      if (diag && row_ok && n - dl >= 0) ss[t] = fmaf(c * sGain[j], raw, HAS_SE ? sTw[i * TS + j] : sBias[j]);
    }
  }

  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < 12; ++e) mx = fmaxf(mx, sd[e]);
#pragma unroll
  for (int t = 0; t < kMaxSparse; ++t) mx = fmaxf(mx, ss[t]);
  mx = col_max(mx);
  if (mx == -INFINITY) mx = 0.f;  // row past N
  float lsum = 0.f;
#pragma unroll
  for (int e = 0; e < 12; ++e) { sd[e] = __expf(sd[e] - mx); lsum += sd[e]; }
#pragma unroll
  for (int t = 0; t < kMaxSparse; ++t) { ss[t] = __expf(ss[t] - mx); lsum += ss[t]; }
  lsum = col_sum(lsum);
  const long long rowbase = ((long long)b * p.H + h) * N;
  if (row_ok && g == 0 && p.lse) p.lse[rowbase + n] = mx + __logf(lsum);
  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const float inv = row_ok ? a / lsum : 0.f;
#pragma unroll
  for (int e = 0; e < 12; ++e) sd[e] *= inv;
#pragma unroll
  for (int t = 0; t < kMaxSparse; ++t) ss[t] *= inv;

  f32x4_t accO[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) accO[db] = zero4();
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    const s16x4_t pb = pack_bf16x4(sd[4 * kk], sd[4 * kk + 1], sd[4 * kk + 2], sd[4 * kk + 3]);
    const bf16_t* vr = sV + (16 * w + 16 * kk + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
    for (int db = 0; db < DB; ++db) accO[db] = mfma_16x16x16(lds_read_tr16(vr + 16 * db), pb, accO[db]);
  }

  // Long-range taps: V rows [n0 - delta, n0 - delta + 64) through a double-buffered LDS block.
  uint4 stg[CH];
  if (NS > 0) stage_rows<CH, CPR>(stg, vb, p.vs.n, n0 - p.taps.delta[W + 1], N, tid);
#pragma unroll
  for (int t = 0; t < kMaxSparse; ++t) {
    if (t < NS) {
      bf16_t* buf = sVs[t & 1];
#pragma unroll
      for (int cI = 0; cI < CH; ++cI) {
        const int chunk = tid + cI * kBlock;
        const int r = chunk / CPR, cc = chunk - r * CPR;
        st16(buf + r * RV + cc * 8, stg[cI]);
      }
      __syncthreads();
      if (t + 1 < NS) stage_rows<CH, CPR>(stg, vb, p.vs.n, n0 - p.taps.delta[W + 2 + t], N, tid);
      const float pt = ss[t];  // zero outside the diagonal lane
      const int e = i & 3;
      const s16x4_t bd = pack_bf16x4(e == 0 ? pt : 0.f, e == 1 ? pt : 0.f, e == 2 ? pt : 0.f,
                                     e == 3 ? pt : 0.f);
      const bf16_t* vr = buf + (16 * w + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db) accO[db] = mfma_16x16x16(lds_read_tr16(vr + 16 * db), bd, accO[db]);
    }
  }

  if (row_ok) {
    bf16_t* ob = static_cast<bf16_t*>(p.out) + b * p.os.b + h * p.os.h + n * p.os.n + 4 * g;
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<uint2*>(ob + 16 * db) =
          pack_bf16x4_u2(accO[db][0], accO[db][1], accO[db][2], accO[db][3]);
  }
}

template <int D>
static hipError_t launch_fwd_mfma_d(const FwdParams& p0, hipStream_t st) {
  FwdParams p = p0;
  p.n_tiles = (p.N + 63) / 64;
  const long long nblocks = (long long)p.B * p.H * p.n_tiles;
  if (nblocks == 0) return hipSuccess;
  if (p.scale_embed)
    hipLaunchKernelGGL((fwd_mfma_kernel<D, true>), dim3((unsigned)nblocks), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL((fwd_mfma_kernel<D, false>), dim3((unsigned)nblocks), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

bool fwd_mfma_supported(int D, const TapTable& t) {
  return (D == 32 || D == 64 || D == 128) && t.J - t.W - 1 <= kMaxSparse;
}

hipError_t launch_fwd_mfma(const FwdParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return launch_fwd_mfma_d<32>(p, st);
    case 64: return launch_fwd_mfma_d<64>(p, st);
    case 128: return launch_fwd_mfma_d<128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsqg
