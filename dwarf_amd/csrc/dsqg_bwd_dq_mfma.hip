// DSQG backward, launch 1, bf16 MFMA path (gfx950): query-centric dq, D' and the per-workgroup
// parameter-gradient partials.
//
// A workgroup owns one (b,h) and a run of 64-row query tiles; wave w owns rows n0+16w .. +15 of
// the tile.  With lse from the forward, every weight alpha_j = exp(s_j - lse) is known as soon
// as its score is, so the taps stream through once:
//   u_j   = dOut . v_j                      (U^T = V dOut^T on the MFMA, like S^T = K Q^T)
//   D'   += alpha_j u_j
//   X    += g_j alpha_j (u_j - D0) k_j,   Y += g_j alpha_j k_j   (K^T from LDS, ds_read_tr16_b64)
// and at the end dq = c (a (X - (D' - D0) Y) + sum_j dS_j se_j) with dS_j = a alpha_j (u_j - D').
// This is sum_j dS_j (c g_j k_j + c se_j), the gradient of s_j = c g_j q.k_j + b_j + c q.se_j.
// D0, the dense band's alpha-weighted mean of u, is known before the first product; taking it
// out of u before the bf16 rounding of the operands keeps their error proportional to u - D'.
// The dense band and the long-range taps are laid out as in the forward (dsqg_fwd_mfma.hip):
// band keys [n0w-32, n0w+16) as three 16x16 tiles, long-range taps as the diagonal of one tile.
// dS is then written to a per-wave [query][tap] table in LDS, from which the workgroup sums
// dbias (and dg, da) in a fixed order and dse = c sum_q dS q runs on the MFMA (Q^T dS over
// the tile's 64 queries, its [D x J] output tiles split over the four waves).
// With scale_embed the q.se_j term is an MFMA (SE Q^T): for the dense taps filed in a per-wave
// [query][tap] table that shares the wave's staging block, for the long-range taps in their dS
// table slots until the diagonal lane reads them.  scale_embed is staged as two bf16 planes
// (hi = bf16(se), lo = bf16(se - hi)), and every weight that enters an MFMA (the dense band's
// and the one-hot long-range X / Y weights, dS in dse and in SE^T dS^T) is split the same way,
// so these products keep fp32 precision as in the reference (kernels/dsqg_attention_v3.py:
// 257-271 sums dq and dse in fp32).
//
// Every long-range pair's dk/dv weights, bf16(c g_j dS_j) and bf16(a alpha_j), also go to the
// workspace ([b,h][tap][query] dwords) for launch 2, so that the key-centric pass needs no
// long-range score, lse or D' of its own.
//
// Follows _compute_D_v3 + _bwd_dq_v3 (kernels/dsqg_attention_v3.py:170-275), except that D' is
// computed from the fp32 weights and the parameter gradients avoid atomics.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_mfma.hpp"

namespace dsqg {

// Row stride of the per-wave [query][tap] tables (floats; 16 B aligned rows, 48 taps).  52
// rather than 48: the column reads of the dse product (rows 4g + 0..3, column i), the diagonal
// lanes' long-range entries (row i, one column) and the band's dS writes then fall on distinct
// banks (or two to a bank) instead of four to a bank.
constexpr int kDqTableStride = 52;

// DG: the score gain's gradient is requested (its c q.k table in dynamic LDS and the extra row
// sums are compiled in only then).
template <int D, bool HAS_SE, int NSC, bool DG>
__global__ __launch_bounds__(kBlock, D == 128 ? 1 : (D > 64 || (HAS_SE && NSC != 11) ? 2 : 3)) void bwd_dq_mfma_kernel(BwdParams p) {
  using G_ = Geo<D>;
  constexpr int QT = 64;
  constexpr int KS = G_::KS;
  constexpr int DB = G_::DB;
  constexpr int RV = G_::RV;              // LDS row stride (36 dwords at D=64: conflict-free 16-byte row reads)
  constexpr int WIN = QT + kMaxWindow;
  constexpr int CPR = G_::CPR;
  constexpr int CPS = G_::CPS;            // chunks per staged (padded) row
  constexpr int CWIN = (WIN * CPS + kBlock - 1) / kBlock;
  constexpr int CHW = G_::CHW;            // 16-byte chunks per lane of a wave's 16-row block
  constexpr int CPRP = G_::CPRP;          // lanes per row in the row-chunk layout
  constexpr int NSM = NSC > 0 ? NSC : kMaxSparse;
  constexpr int PF = 2;                   // long-range K/V operands loaded ahead of use
  constexpr int TS = kDqTableStride;
  constexpr int TST = 38;                 // row stride of the dense-tap T table (2-way bank reads)
  constexpr int KSB = (16 * RV > 32 * TST ? 16 * RV : 32 * TST);  // bf16 per wave staging block
  constexpr int SEJ = 48;                 // scale_embed rows staged (J <= 48)
  constexpr int NTSE = 3 * DB;            // 16x16 tiles of dse^T [D x 48]
  constexpr int TPW = (NTSE + 3) / 4;     // ... per wave
  constexpr float kLog2e = 1.4426950408889634f;

  __shared__ __align__(16) bf16_t sK[WIN * RV];        // dense-window K rows
  __shared__ __align__(16) bf16_t sV[WIN * RV];        // dense-window V rows
  // Wave-private staging block: with scale_embed first the dense-tap table
  // T[i][j] = log2e (bias_j + c q_i.se_j), then the long-range K rows, then the wave's Q rows
  // (read by every wave for dse).
  __shared__ __align__(16) bf16_t sKs[4][HAS_SE ? KSB : 16 * RV];
  // scale_embed rows as two bf16 planes, hi = bf16(se) and lo = bf16(se - hi): q.se and
  // SE^T dS then carry se to about 2^-17 relative, as the fp32 se of the reference.
  __shared__ __align__(16) bf16_t sSE[HAS_SE ? SEJ * RV : 8];
  __shared__ __align__(16) bf16_t sSElo[HAS_SE ? SEJ * RV : 8];
  // dS[query][tap] per wave; with scale_embed it lives in the V window once the band is done
  // (D >= 64), which leaves room for three workgroups per CU.
  constexpr bool TBL_IN_V = HAS_SE && WIN * RV * 2 >= 4 * 16 * TS * 4;
  __shared__ __align__(16) float sDSst[TBL_IN_V ? 4 : 4 * 16 * TS];
  // c q.k per (query, tap), for dg only: dynamic LDS, present when score_gain's gradient is
  // requested (without it the workgroup fits three per CU).
  extern __shared__ __align__(16) float sDyn[];
  float* const sRAW = sDyn;
  __shared__ float sBias2[kMaxTaps];
  __shared__ float sGain[kMaxTaps];
  // Per wave, one long-range tap's row results (q.k, dOut.v).
  __shared__ __align__(16) float sPair[4][16][2];

  const int tid = threadIdx.x;
  // The kernel arguments of the prologue in one round trip: sizes and input strides pass through
  // an empty asm statement that the code after it depends on, the input pointers are its
  // operands, so all are requested before it and waited for once (otherwise the grid constants
  // come first, the block-number divisions wait for them, and each later group of arguments
  // costs another dependent round trip).
  int nblk = (int)gridDim.x;
  asm volatile("" : "+s"(nblk), "+s"(p.H), "+s"(p.N), "+s"(p.n_chunks), "+s"(p.taps.J), "+s"(p.taps.W),
               "+s"(p.qs.b), "+s"(p.qs.h), "+s"(p.qs.n), "+s"(p.ks.b), "+s"(p.ks.h), "+s"(p.ks.n),
               "+s"(p.vs.b), "+s"(p.vs.h), "+s"(p.vs.n), "+s"(p.dos.b), "+s"(p.dos.h), "+s"(p.dos.n)
               : "s"(p.q), "s"(p.k), "s"(p.v), "s"(p.dout), "s"(p.lse), "s"(p.pos_bias), "s"(p.if_gain));
  const int lb = xcd_logical_block(blockIdx.x, nblk);
  const int bh = lb / p.n_chunks, chunk = lb - bh * p.n_chunks;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const int NS = NSC > 0 ? NSC : J - W - 1;
  const float c = p.scale, c2 = p.scale * kLog2e;
  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const bool se_grad = p.part_se != nullptr;
  constexpr bool g_grad = DG;
  const int qsn = (int)p.qs.n, ksn = (int)p.ks.n, vsn = (int)p.vs.n, dosn = (int)p.dos.n;

  const __amdgpu_buffer_rsrc_t rQ = slice_rsrc(static_cast<const bf16_t*>(p.q) + b * p.qs.b + h * p.qs.h, p.qs.n, N, D);
  const __amdgpu_buffer_rsrc_t rK = slice_rsrc(static_cast<const bf16_t*>(p.k) + b * p.ks.b + h * p.ks.h, p.ks.n, N, D);
  const __amdgpu_buffer_rsrc_t rV = slice_rsrc(static_cast<const bf16_t*>(p.v) + b * p.vs.b + h * p.vs.h, p.vs.n, N, D);
  const __amdgpu_buffer_rsrc_t rO = slice_rsrc(static_cast<const bf16_t*>(p.dout) + b * p.dos.b + h * p.dos.h, p.dos.n, N, D);
  bf16_t* dqb = static_cast<bf16_t*>(p.dq) + b * p.dqs.b + h * p.dqs.h;
  const long long rowbase = ((long long)b * p.H + h) * N;

  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, i = l & 15, g = l >> 4;
  const int qlane = opaque(i * qsn + 8 * g), olane = opaque(i * dosn + 8 * g);
  // Row-chunk layout (whole rows per D/8 lanes) for the long-range rows and their dot partners.
  int qlaneR[CHW], olaneR[CHW], klaneR[CHW], vlaneR[CHW];
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    qlaneR[u] = opaque(rc_lane<D>(l, u, qsn));
    olaneR[u] = opaque(rc_lane<D>(l, u, dosn));
    klaneR[u] = opaque(rc_lane<D>(l, u, ksn));
    vlaneR[u] = opaque(rc_lane<D>(l, u, vsn));
  }

  // Per-tap bias and gain (J <= kMaxTaps < kBlock: one per thread).  With scale_embed they are
  // staged here, with the scale_embed rows, all requested before the one wait: held in registers
  // across the tile's loads instead, they cost that kernel three spilled registers and 1.3 us.
  // Without it they are requested after the window rows and stored just before the first
  // barrier, which waits for those rows anyway.  (Stored before any tile load was issued, their
  // wait held back every load of the workgroup by a memory round trip.)
  const int jc = tid < J ? tid : J - 1;
  [[maybe_unused]] float bias_ld = 0.f, gain_ld = 1.f;
  if constexpr (HAS_SE) {
    bias_ld = p.pos_bias[jc * p.H + h];
    gain_ld = p.score_gain ? p.score_gain[h * J + jc] : 1.0f;
    SeRows<D> seR;
    seR.load(p.scale_embed, J, tid);
    if (tid < J) {
      sBias2[tid] = bias_ld * kLog2e;
      sGain[tid] = gain_ld;
    }
    seR.template store<RV>(sSE, sSElo, tid);
  }

  float* const sDS = TBL_IN_V ? reinterpret_cast<float*>(sV) : sDSst;
  // Table columns J..47 are read as zeros (whole 4-wide groups feed the MFMA operands); a table
  // in the V window gets them after the band.
  // Thread t clears row t % 64 from column J + t / 64 on, every fourth column.
  for (int j = J + (tid >> 6); j < 48; j += kBlock / 64) {
    if (!TBL_IN_V) sDS[(tid & 63) * TS + j] = 0.f;
    if (g_grad) sRAW[(tid & 63) * TS + j] = 0.f;
  }

  float acc_bias = 0.f, acc_gain = 0.f, acc_if = 0.f;
  f32x4_t accSE[HAS_SE ? TPW : 1];  // this wave's dse^T tiles w, w+4, ...
#pragma unroll
  for (int k = 0; k < (HAS_SE ? TPW : 1); ++k) accSE[k] = zero4();

  float* sDSw = sDS + w * 16 * TS;
  float* sRAWw = sRAW + w * 16 * TS;  // dereferenced only when g_grad
  // The wave's 16 values of D' go through its own hand-off block once the tap loop is over.
  float* sDpw = &sPair[w][0][0];
  bf16_t* sKsw = sKs[w];
  float* sTw = reinterpret_cast<float*>(sKsw);
  const int t_begin = chunk * p.tiles_per_block;
  // Without scale_embed the plan gives one tile per workgroup (checked at launch): a loop of
  // one trip keeps the compiler from holding loop-invariant addresses across tiles.
  const int t_end = t_begin + 1;
  int dl_s[NSM];
  load_sparse_deltas(p.taps, dl_s);

  for (int tile = t_begin; tile < t_end; ++tile) {
    const int n0 = tile * QT;
    const int n0w = n0 + 16 * w;
    const int n = n0w + i;
    const bool row_ok = n < N;

    // ---- Loads (zero outside [0, N)). ----
    // Dense window K and V rows [n0-32, n0+64), staged once per workgroup in LDS.
    uint4 wk[CWIN], wv[CWIN];
#pragma unroll
    for (int u = 0; u < CWIN; ++u) {
      const int ci = tid + u * kBlock;
      const bool cv = ci % CPS < CPR;
      wk[u] = bload16(rK, (n0 - kMaxWindow) * ksn + opaque(cv ? (ci / CPS) * ksn + (ci % CPS) * 8 : kNoElem));
      wv[u] = bload16(rV, (n0 - kMaxWindow) * vsn + opaque(cv ? (ci / CPS) * vsn + (ci % CPS) * 8 : kNoElem));
    }
    if constexpr (!HAS_SE) {
      bias_ld = p.pos_bias[jc * p.H + h];
      gain_ld = p.score_gain ? p.score_gain[h * J + jc] : 1.0f;
    }
    bf16x8_t qB[KS], oB[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bool sv = 8 * g + 32 * s < D;  // the zero columns of D = 80's last K-step
      qB[s] = as_bf16x8(bload16(rQ, n0w * qsn + (sv ? qlane + 32 * s : kNoElem)));
      oB[s] = as_bf16x8(bload16(rO, n0w * dosn + (sv ? olane + 32 * s : kNoElem)));
    }
    uint4 qR[CHW], oR[CHW];
#pragma unroll
    for (int u = 0; u < CHW; ++u) {
      qR[u] = bload16(rQ, n0w * qsn + qlaneR[u]);
      oR[u] = bload16(rO, n0w * dosn + olaneR[u]);
    }
    // Unconditional (a row past N reads row N - 1 and is masked below): a load under the row
    // test was waited for inside the branch, before the long-range loads could be issued.
    const float lse_ld = p.lse[rowbase + (row_ok ? n : N - 1)];
    // Long-range K/V rows n0w - delta + 0..15, whole rows per D/8 lanes, PF taps ahead.
    uint4 kS[PF][CHW], vS[PF][CHW];
#pragma unroll
    for (int t = 0; t < PF; ++t) {
      if (t < NS) {
        const int m0 = n0w - dl_s[t];
#pragma unroll
        for (int u = 0; u < CHW; ++u) {
          kS[t][u] = bload16(rK, m0 * ksn + klaneR[u]);
          vS[t][u] = bload16(rV, m0 * vsn + vlaneR[u]);
        }
      }
    }

    if (!HAS_SE && tid < J) {
      sBias2[tid] = bias_ld * kLog2e;
      sGain[tid] = gain_ld;
    }

    __syncthreads();  // previous tile's readers of sK / tables are done
#pragma unroll
    for (int u = 0; u < CWIN; ++u) {
      const int ci = tid + u * kBlock;
      if (ci < WIN * CPS) {
        st16(sK + (ci / CPS) * RV + (ci % CPS) * 8, wk[u]);
        st16(sV + (ci / CPS) * RV + (ci % CPS) * 8, wv[u]);
      }
    }
    __syncthreads();

    // ---- Dense band: S^T = K Q^T, U^T = V dOut^T. ----
    f32x4_t accS[3], accU[3];
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
      accS[kk] = zero4();
      accU[kk] = zero4();
      const bf16_t* kr = sK + (16 * w + 16 * kk + i) * RV + 8 * g;
      const bf16_t* vr = sV + (16 * w + 16 * kk + i) * RV + 8 * g;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        accS[kk] = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(kr + 32 * s)), qB[s], accS[kk]);
        accU[kk] = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(vr + 32 * s)), oB[s], accU[kk]);
      }
    }
    if constexpr (HAS_SE) {
#pragma unroll
      for (int jb = 0; jb < 3; ++jb) {
        f32x4_t acc = zero4();
        const bf16_t* sr = sSE + (16 * jb + i) * RV + 8 * g;
        const bf16_t* srl = sSElo + (16 * jb + i) * RV + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          acc = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(sr + 32 * s)), qB[s], acc);
          acc = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(srl + 32 * s)), qB[s], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jb + 4 * g + r;
          if (j <= W) sTw[i * TST + j] = fmaf(c2, acc[r], sBias2[j]);
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);
      __builtin_amdgcn_wave_barrier();
    }

    // Dense weights first; D0 = the band's weighted mean of u is subtracted from u before the
    // bf16 rounding of the dQ operands, so their error scales with u - D' rather than u.
    float al[12], uu[12];
    float dlane = 0.f, wlane = 0.f;
    const int dl0 = 32 - 4 * g + i;
    const float lse2 = row_ok ? lse_ld * kLog2e : 0.f;
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int dl = dl0 - 16 * kk - r;
        const bool ok = row_ok && (unsigned)dl <= (unsigned)W && n >= dl;
        const int j = ok ? dl : 0;
        const float s2 = fmaf(sGain[j] * c2, accS[kk][r], HAS_SE ? sTw[i * TST + j] : sBias2[j]);
        const float alpha = ok ? __builtin_amdgcn_exp2f(s2 - lse2) : 0.f;
        al[4 * kk + r] = alpha;
        uu[4 * kk + r] = accU[kk][r];
        dlane = fmaf(alpha, accU[kk][r], dlane);
        wlane += alpha;
        // c q.k for dg goes to the table now (frees the score registers for the taps loop).
        if (g_grad && (unsigned)dl <= (unsigned)W) sRAWw[i * TS + dl] = c * accS[kk][r];
      }
    }
    const float wsum = col_sum(wlane);
    const float D0 = wsum > 0.f ? col_sum(dlane) / wsum : 0.f;
    if constexpr (TBL_IN_V) {
      __syncthreads();  // every wave's band reads of sV are done: the dS tables move in
      for (int j = J + g; j < 48; j += 4) sDSw[i * TS + j] = 0.f;
    }
    if constexpr (HAS_SE) {
      // T for the long-range taps (log2e (bias_j + c q.se_j), the same MFMA as the dense taps'
      // table) waits in the taps' dS table slots until the diagonal lane reads it in the taps
      // loop; dS overwrites it after the loop.
#pragma unroll
      for (int jb = 0; jb < 3; ++jb) {
        if (16 * jb + 15 <= W) continue;
        f32x4_t acc = zero4();
        const bf16_t* sr = sSE + (16 * jb + i) * RV + 8 * g;
        const bf16_t* srl = sSElo + (16 * jb + i) * RV + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          acc = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(sr + 32 * s)), qB[s], acc);
          acc = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(srl + 32 * s)), qB[s], acc);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = 16 * jb + 4 * g + r;
          if (j > W && j < J) sDSw[i * TS + j] = fmaf(c2, acc[r], sBias2[j]);
        }
      }
    }
    f32x4_t X[DB], Y[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) { X[db] = zero4(); Y[db] = zero4(); }
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
      float ga[4], gau[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int dl = dl0 - 16 * kk - r;
        const int j = (unsigned)dl <= (unsigned)W ? dl : 0;
        ga[r] = sGain[j] * al[4 * kk + r];
        gau[r] = ga[r] * (uu[4 * kk + r] - D0);
      }
      // The weights as bf16 hi + lo pairs: the products keep the weights' fp32 precision.
      s16x4_t b1, b1l, b2, b2l;
      split_bf16x4(gau[0], gau[1], gau[2], gau[3], b1, b1l);
      split_bf16x4(ga[0], ga[1], ga[2], ga[3], b2, b2l);
      const bf16_t* kr = sK + (16 * w + 16 * kk + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const s16x4_t at = lds_read_tr16(kr + 16 * db);
        X[db] = mfma_16x16x16(at, b1, X[db]);
        X[db] = mfma_16x16x16(at, b1l, X[db]);
        Y[db] = mfma_16x16x16(at, b2, Y[db]);
        Y[db] = mfma_16x16x16(at, b2l, Y[db]);
      }
    }

    // ---- Long-range taps (diagonal of one 16x16 tile each). ----
    const bool diag = g == (i >> 2);
    const uint2 ohm = onehot_masks(i & 3);
    const bf16_t* ksr = sKsw + (4 * g + (i >> 2)) * RV + 4 * (i & 3);
    float als[NSM], uus[NSM];
#pragma unroll
    for (int t = 0; t < NSM; ++t) {
      als[t] = 0.f; uus[t] = 0.f;
      if (NSC > 0 || t < NS) {
        const int j = W + 1 + t;
        // q.k and dOut.v on the VALU: each lane dots its 16-byte chunk, the row's lanes sum
        // (DPP), and one lane per row hands the results to the diagonal lane through LDS.  The
        // key rows are staged (natural row order) for the transposing reads of X and Y.
#pragma unroll
        for (int u = 0; u < CHW; ++u) {
          const float qk = group_sum<CPRP>(dot8_bf16(qR[u], kS[t % PF][u], 0.f));
          const float dv = group_sum<CPRP>(dot8_bf16(oR[u], vS[t % PF][u], 0.f));
          if (rc_valid<D>(l, u)) st16(sKsw + rc_row<D>(l, u) * RV + rc_chunk<D>(l, u) * 8, kS[t % PF][u]);
          if (rc_chunk<D>(l, u) == 0)
            *reinterpret_cast<float2*>(sPair[w][rc_row<D>(l, u)]) = float2{qk, dv};
        }
        if (t + PF < NS) {
          const int m0 = n0w - dl_s[t + PF];
#pragma unroll
          for (int u = 0; u < CHW; ++u) {
            kS[t % PF][u] = bload16(rK, m0 * ksn + klaneR[u]);
            vS[t % PF][u] = bload16(rV, m0 * vsn + vlaneR[u]);
          }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): staged rows and pairs are written
        __builtin_amdgcn_wave_barrier();
        const float2 pr = *reinterpret_cast<const float2*>(sPair[w][i]);
        const float raw = pr.x, uval = pr.y;
        const float s2 = fmaf(sGain[j] * c2, raw, HAS_SE ? sDSw[i * TS + j] : sBias2[j]);
        const bool ok = diag && row_ok && n >= dl_s[t];
        const float alpha = ok ? __builtin_amdgcn_exp2f(s2 - lse2) : 0.f;
        als[t] = alpha;
        uus[t] = uval;
        if (g_grad && diag) sRAWw[i * TS + j] = c * raw;
        dlane = fmaf(alpha, uval, dlane);
        const float gal = sGain[j] * alpha;
        // One-hot weights as bf16 hi + lo pairs: the products keep the weights' fp32 precision.
        s16x4_t b1, b1l, b2, b2l;
        // With scale_embed they are placed by per-lane element masks (fewer instructions; that
        // variant then fits without spills), without by 64-bit shifts (no extra registers).
        if constexpr (HAS_SE) {
          split_onehot_bf16x4(gal * (uval - D0), ohm, b1, b1l);
          split_onehot_bf16x4(gal, ohm, b2, b2l);
        } else {
          split_onehot_bf16x4(gal * (uval - D0), i & 3, b1, b1l);
          split_onehot_bf16x4(gal, i & 3, b2, b2l);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const s16x4_t at = lds_read_tr16(ksr + 16 * db);
          X[db] = mfma_16x16x16(at, b1, X[db]);
          X[db] = mfma_16x16x16(at, b1l, X[db]);
          Y[db] = mfma_16x16x16(at, b2, Y[db]);
          Y[db] = mfma_16x16x16(at, b2l, Y[db]);
        }
      }
    }

    const float Dp = col_sum(dlane);  // D' = dOut . o (pre-gain o) for query n
    if constexpr (HAS_SE) {
      // The wave's Q rows (natural order) replace its K rows, for dse after the tables are done.
      if (se_grad) {
#pragma unroll
        for (int u = 0; u < CHW; ++u)
          if (rc_valid<D>(l, u)) st16(sKsw + rc_row<D>(l, u) * RV + rc_chunk<D>(l, u) * 8, qR[u]);
      }
    }

    // ---- dS table [query][tap] (every entry j < J is written: zero where masked). ----
#pragma unroll
    for (int kk = 0; kk < 3; ++kk)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int dl = dl0 - 16 * kk - r;
        if ((unsigned)dl <= (unsigned)W) {
          const float dS = a * al[4 * kk + r] * (uu[4 * kk + r] - Dp);
          sDSw[i * TS + dl] = dS;
        }
      }
    if (diag) {
      // The long-range taps' dk/dv weights go to the workspace for launch 2, which then needs
      // neither the taps' dot products nor their queries' lse and D': [b,h][tap][query] dwords
      // holding bf16(c g_j dS_j) (low half) and bf16(a alpha_j) (high half), zero for a masked tap.
      unsigned* const lw = reinterpret_cast<unsigned*>(p.lrw) + (long long)bh * NS * N + n;
#pragma unroll
      for (int t = 0; t < NSM; ++t)
        if (NSC > 0 || t < NS) {
          const float ds = a * als[t] * (uus[t] - Dp);
          sDSw[i * TS + W + 1 + t] = ds;
          if (row_ok) lw[(long long)t * N] = cvt_pk_bf16(c * sGain[W + 1 + t] * ds, a * als[t]);
        }
    }
    if (g == 0) sDpw[i] = row_ok ? Dp : 0.f;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();

    // dq = c (a (X - D' Y) + SE^T dS^T): c a X - c a (D' - D0) Y, plus SE^T (c dS)^T.
    f32x4_t dQ[DB];
    const float ca = c * a, cad = ca * (Dp - D0);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) dQ[db][r] = fmaf(ca, X[db][r], -cad * Y[db][r]);
    if constexpr (HAS_SE) {
#pragma unroll
      for (int jb = 0; jb < 3; ++jb) {
        const float4 d4 = *reinterpret_cast<const float4*>(sDSw + i * TS + 16 * jb + 4 * g);
        s16x4_t bs, bsl;
        split_bf16x4(c * d4.x, c * d4.y, c * d4.z, c * d4.w, bs, bsl);
        const int so = (16 * jb + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const s16x4_t sh = lds_read_tr16(sSE + so + 16 * db);
          dQ[db] = mfma_16x16x16(sh, bs, dQ[db]);
          dQ[db] = mfma_16x16x16(sh, bsl, dQ[db]);
          dQ[db] = mfma_16x16x16(lds_read_tr16(sSElo + so + 16 * db), bs, dQ[db]);
        }
      }
    }
    // dq (MFMA layout: lane (i, g) holds query i, d = 16 db + 4 g + 0..3) leaves as whole rows
    // through a wave-private LDS block (the K staging block; with scale_embed it holds the Q
    // rows for dse, and the wave's rows of the K window, free since the barrier after the band,
    // take its place), then 16-byte row pieces per lane.  Without a free block (scale_embed at
    // D = 32, whose tables stay outside the V window) the quads are stored directly.
    if constexpr (!HAS_SE || TBL_IN_V) {
      bf16_t* const stg = HAS_SE ? sK + 16 * w * RV : sKsw;
#pragma unroll
      for (int db = 0; db < DB; ++db)
        *reinterpret_cast<uint2*>(stg + i * RV + 16 * db + 4 * g) =
            pack_bf16x4_u2(dQ[db][0], dQ[db][1], dQ[db][2], dQ[db][3]);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the rows are staged
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int u = 0; u < CHW; ++u) {
        const int rr = rc_row<D>(l, u), cc = rc_chunk<D>(l, u);
        if (n0w + rr < N && cc < CPR)
          st16(dqb + (n0w + rr) * p.dqs.n + 8 * cc, *reinterpret_cast<const uint4*>(stg + rr * RV + 8 * cc));
      }
    } else if (row_ok) {
      bf16_t* o = dqb + n * p.dqs.n + 4 * g;
#pragma unroll
      for (int db = 0; db < DB; ++db)
        *reinterpret_cast<uint2*>(o + 16 * db) =
            pack_bf16x4_u2(dQ[db][0], dQ[db][1], dQ[db][2], dQ[db][3]);
    }
    if (row_ok && g == 0) p.dpre[rowbase + n] = Dp;

    // dbias / dg column sums of this wave's 16 table rows (its own writes, complete above),
    // and the wave's sum of D' (for da): no workgroup barrier inside the tile.
    if (l < J) {
      float sb = 0.f, sg = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float ds = sDSw[r * TS + l];
        sb += ds;
        if (g_grad) sg = fmaf(ds, sRAWw[r * TS + l], sg);
      }
      acc_bias += sb;
      acc_gain += sg;
    }
    if (l == 0) {
      float sa = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) sa += sDpw[r];
      acc_if += sa;
    }
    if constexpr (HAS_SE) __syncthreads();  // all waves' tables (and Q rows) are complete
    // dse partial on the MFMA: dSE^T (d x j) += Q^T (d x q) dS (q x j) over the tile's 64
    // queries; wave w owns the output tiles w, w+4, ... of the 3 x DB grid.
    if constexpr (HAS_SE) {
      if (se_grad) {
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
          const int idx = w + 4 * k;
          if (idx < NTSE) {
            const int jb = idx / DB, db = idx - jb * DB;
#pragma unroll
            for (int ww = 0; ww < 4; ++ww) {
              const float* col = sDS + (ww * 16 + 4 * g) * TS + 16 * jb + i;
              s16x4_t bs, bsl;
              split_bf16x4(col[0], col[TS], col[2 * TS], col[3 * TS], bs, bsl);
              const bf16_t* qr = sKs[ww] + (4 * g + (i >> 2)) * RV + 4 * (i & 3) + 16 * db;
              const s16x4_t qt = lds_read_tr16(qr);
              accSE[k] = mfma_16x16x16(qt, bs, accSE[k]);
              accSE[k] = mfma_16x16x16(qt, bsl, accSE[k]);
            }
          }
        }
      }
    }
  }

  // The four waves' partial sums meet in their own (now free) table blocks; one partial row per
  // workgroup, summed in wave order.
  {
    if constexpr (HAS_SE) __syncthreads();  // the last tile's dse reads of every wave's table are done
    float* red = sDSw;  // wave-private until the barrier
    if (l < J) { red[l] = acc_bias; red[64 + l] = acc_gain; }
    if (l == 0) red[128] = acc_if;
    __syncthreads();
    if (tid < J) {
      float sb = 0.f, sg = 0.f;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        sb += sDS[ww * 16 * TS + tid];
        sg += sDS[ww * 16 * TS + 64 + tid];
      }
      p.part_bias[(long long)lb * J + tid] = sb;
      if (g_grad) p.part_gain[(long long)lb * J + tid] = sg;
    }
    if (tid == 0 && p.part_if) {
      float sa = 0.f;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) sa += sDS[ww * 16 * TS + 128];
      p.part_if[lb] = sa;
    }
  }
  if constexpr (HAS_SE) {
    if (se_grad) {
      // Lane (i, g) of tile (jb, db) holds dSE^T[d = 16 db + 4 g + r][j = 16 jb + i], r = 0..3.
#pragma unroll
      for (int k = 0; k < TPW; ++k) {
        const int idx = w + 4 * k;
        const int jb = idx / DB, db = idx - jb * DB;
        const int j = 16 * jb + i;
        if (idx < NTSE && j < J)
          *reinterpret_cast<float4*>(p.part_se + ((long long)lb * J + j) * D + 16 * db + 4 * g) =
              make_float4(c * accSE[k][0], c * accSE[k][1], c * accSE[k][2], c * accSE[k][3]);
      }
    }
  }
}

template <int D, bool HAS_SE>
static void launch_dq_mfma_ns(const BwdParams& p, unsigned nb, hipStream_t st) {
  if (p.part_gain) {  // the score gain's gradient: the generic-table form with its dg table
    const size_t dyn = sizeof(float) * 4 * 16 * kDqTableStride;
    hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 0, true>), dim3(nb), dim3(kBlock), dyn, st, p);
    return;
  }
  switch (p.taps.J - p.taps.W - 1) {
    case 11: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 11, false>), dim3(nb), dim3(kBlock), 0, st, p); break;
    case 13: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 13, false>), dim3(nb), dim3(kBlock), 0, st, p); break;
    case 14: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 14, false>), dim3(nb), dim3(kBlock), 0, st, p); break;
    default: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 0, false>), dim3(nb), dim3(kBlock), 0, st, p); break;
  }
}

template <int D>
static hipError_t launch_dq_mfma_d(const BwdParams& p, unsigned nb, hipStream_t st) {
  // The scale_embed variant also serves dse requested at se = 0.
  if (p.tiles_per_block != 1) return hipErrorInvalidValue;  // the single-tile form
  if (p.scale_embed || p.part_se) launch_dq_mfma_ns<D, true>(p, nb, st);
  else launch_dq_mfma_ns<D, false>(p, nb, st);
  return hipGetLastError();
}

hipError_t launch_bwd_dq_mfma(const BwdParams& p, int D, unsigned nblocks, hipStream_t st) {
  switch (D) {
    case 32: return launch_dq_mfma_d<32>(p, nblocks, st);
    case 64: return launch_dq_mfma_d<64>(p, nblocks, st);
    case 80: return launch_dq_mfma_d<80>(p, nblocks, st);
    case 96: return launch_dq_mfma_d<96>(p, nblocks, st);
    case 128: return launch_dq_mfma_d<128>(p, nblocks, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsqg
