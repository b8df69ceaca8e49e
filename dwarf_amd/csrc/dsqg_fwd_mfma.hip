// DSQG forward, bf16 MFMA path (gfx950).
//
// Workgroup = one (b,h) and 64 query rows [n0, n0+64); wave w owns rows n0+16w .. +15.
//  1. The dense window, K/V rows [n0-32, n0+64), is copied once into LDS (zero rows outside
//     [0,N)).  Each wave's queries see the 48-key band [n0w-32, n0w+16) of it.
//  2. Scores for the band: S^T = K_band Q^T with v_mfma_f32_16x16x32_bf16 (A = key rows from
//     LDS, B = the wave's query rows, straight from global memory).  Lane l then holds query
//     column i = l%16 and keys 4*(l/16) + r of each 16-key block, i.e. delta = n - m is known
//     per register; taps outside delta in [0, W] (or before row 0) become -inf.
//  3. Long-range taps: for tap delta the key rows are the contiguous block n0w - delta + 0..15.
//     They are loaded in the row-chunk layout (8 lanes x 16 bytes per 128-byte row at D = 64,
//     4 lanes x 48 bytes per 192-byte row at D = 96) and dotted with
//     the query rows on the VALU (v_dot2_f32_bf16, DPP sum over the row's lanes); the 16 scores
//     go through a per-wave LDS table to the lane that owns query i's taps.  An MFMA diagonal
//     would need the operand order (16 rows x 16 bytes per 16 lanes), which the vector L1
//     serves at about a quarter of the whole-row rate.
//  4. Optional q.se_j term: SE Q^T with the same MFMA for every tap, kept per wave in an LDS
//     table T[i][j] = bias[j] + c q_i . se_j (in the wave's staging block, free until the
//     long-range P V).  se is staged as bf16 hi and lo planes in the window tiles before the
//     window rows arrive, so the term keeps se's fp32 precision.  Without scale_embed T is the
//     bias row.
//  5. Softmax over each query's J taps in registers: the four lanes of a query column combine
//     max and sum with two cross-lane steps; lse = max + log(sum); the weights are normalised
//     (and scaled by the IF gain) before P V.
//     With an alpha_lr buffer the long-range taps' normalised weights are also stored, for the
//     backward ([b,h][tap][query] fp32).
//  6. P V: O^T = V^T P^T with v_mfma_f32_16x16x16_bf16.  Dense taps: V^T from the row-major
//     window tile through ds_read_tr16_b64, P^T already in B layout.  Long-range taps: each
//     tap's 16 V rows (gathered whole-row) are staged in the wave's LDS block and read back the
//     same way, against a one-hot P^T held by the query's diagonal lane.  The output leaves
//     through the same block as 16-byte row stores.
//
// Semantics: _fwd_v3, kernels/dsqg_attention_v3.py:60-163 (plus score gain and IF gain).
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_mfma.hpp"

namespace dsqg {

template <int D, bool HAS_SE, int NSC>
__global__ __launch_bounds__(kBlock, D == 128 ? 1 : (D > 64 ? 3 : (NSC != 11 ? 3 : 4))) void fwd_mfma_kernel(FwdParams p) {
  using G_ = Geo<D>;
  constexpr int QT = 64;                  // query rows per workgroup
  constexpr int KS = G_::KS;              // 16x16x32 steps over the head dim
  constexpr int DB = G_::DB;              // 16-wide head-dim blocks of the output
  constexpr int RV = G_::RV;              // LDS row stride of the K / V tiles (36 dwords at D=64)
  constexpr int WIN = QT + kMaxWindow;    // dense-window rows of V staged in LDS
  constexpr int CPR = G_::CPR;            // 16-byte chunks per row
  constexpr int CPS = G_::CPS;            // ... per staged row (zero chunks pad D = 80 to 96)
  constexpr int CWIN = (WIN * CPS + kBlock - 1) / kBlock;
  constexpr int CHW = G_::CHW;            // chunks per lane of a wave's 16-row block
  constexpr int CPL = G_::CPL;            // ... of one row
  constexpr int NSM = NSC > 0 ? NSC : kMaxSparse;
  // Long-range V blocks held in registers ahead of use.  At D > 64 the register peak lies in the
  // key-row bursts, so four blocks cost no occupancy there (and fewer spills with scale_embed);
  // at D = 64 a fourth block spills.
  constexpr int PF = D > 64 ? 4 : 3;
  constexpr int TS = 49;                  // row stride of the per-wave T table (every tap j < 48; odd: rows on distinct banks)
  constexpr int XB = (16 * RV > 32 * TS ? 16 * RV : 32 * TS);  // bf16 elements per staging block
  constexpr int TR = NSM + (NSM & 1);     // row stride of the long-range score table (distinct banks)
  constexpr float kLog2e = 1.4426950408889634f;

  __shared__ __align__(16) bf16_t sV[WIN * RV];
  __shared__ __align__(16) bf16_t sK[WIN * RV];   // dense-window K rows (MFMA A operands)
  // Wave-private staging block (16 rows x RV): the T table (scale_embed), then each long-range
  // tap's V rows, then the output rows.
  __shared__ __align__(16) bf16_t sVs[4][HAS_SE ? XB : 16 * RV];
  // Per wave: long-range q.k [query][tap], in the wave's staging block (free from the band's
  // query-operand reads to the long-range P V).  With scale_embed the scores are added into the
  // T table instead (its long-range entries are read once, after every tap is scored).
  static_assert(16 * TR * 4 <= 16 * RV * 2, "the score table fits the staging block");
  __shared__ float sBias2[kMaxTaps];   // bias * log2(e)
  __shared__ float sGain2[kMaxTaps];   // gain * c * log2(e)

  const int tid = threadIdx.x;
  // The kernel arguments of the prologue in one round trip: sizes and input strides pass through
  // an empty asm statement that the code after it depends on, the input pointers are its
  // operands, so all are requested before it and waited for once (otherwise the grid constants
  // come first, the block-number divisions wait for them, and each later group of arguments
  // costs another dependent round trip).
  int nblk = (int)gridDim.x;
  asm volatile("" : "+s"(nblk), "+s"(p.H), "+s"(p.N), "+s"(p.n_tiles), "+s"(p.taps.J), "+s"(p.taps.W),
               "+s"(p.qs.b), "+s"(p.qs.h), "+s"(p.qs.n), "+s"(p.ks.b), "+s"(p.ks.h), "+s"(p.ks.n),
               "+s"(p.vs.b), "+s"(p.vs.h), "+s"(p.vs.n)
               : "s"(p.q), "s"(p.k), "s"(p.v), "s"(p.pos_bias), "s"(p.if_gain));
  const int lb = xcd_logical_block(blockIdx.x, nblk);
  const int bh = lb / p.n_tiles, tile = lb - bh * p.n_tiles;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const int NS = NSC > 0 ? NSC : J - W - 1;
  const int n0 = tile * QT;
  const float c2 = p.scale * kLog2e;
  const int qsn = (int)p.qs.n, ksn = (int)p.ks.n, vsn = (int)p.vs.n;
  // The IF gain is requested with the first loads: read after the softmax, it cost every wave a
  // fresh memory round trip, and its wait also held the dense P V for the long-range V prefetch.
  const float if_a = p.if_gain ? p.if_gain[h] : 1.0f;

  const __amdgpu_buffer_rsrc_t rQ = slice_rsrc(static_cast<const bf16_t*>(p.q) + b * p.qs.b + h * p.qs.h, p.qs.n, N, D);
  const __amdgpu_buffer_rsrc_t rK = slice_rsrc(static_cast<const bf16_t*>(p.k) + b * p.ks.b + h * p.ks.h, p.ks.n, N, D);
  const __amdgpu_buffer_rsrc_t rV = slice_rsrc(static_cast<const bf16_t*>(p.v) + b * p.vs.b + h * p.vs.h, p.vs.n, N, D);

  // The wave index is uniform: readfirstlane keeps every row product on the scalar unit.
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, i = l & 15, g = l >> 4;
  const int n0w = n0 + 16 * w;
  const int n = n0w + i;  // query row of this lane's MFMA column
  const bool row_ok = n < N;
  int dl_s[NSM];
  load_sparse_deltas(p.taps, dl_s);

  // ---- Global loads (all zero-filled outside [0, N) by the buffer range check). ----
  // The query rows go first (the band waits for them): with scale_embed the scale_embed rows
  // and the band's B operand (query rows in the MFMA operand order, for the T table), and in
  // both variants the query rows in the row-chunk layout.  Without
  // scale_embed the B operand is read back from that copy, staged in the wave's block after the
  // window barrier (free until the long-range P V), which saves the operand-order global loads
  // (16 rows x 16 B per 16 lanes); with it, the T table needs the operand before the window.
  int qlaneR[CHW], klaneR[CHW];
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    qlaneR[u] = opaque(rc_lane<D>(l, u, qsn));
    klaneR[u] = opaque(rc_lane<D>(l, u, ksn));
  }
  // Per-tap bias and gain (J <= kMaxTaps < kBlock: one per thread), stored to LDS below after a
  // wait that must cover as few loads as possible: with scale_embed they go first, with the
  // scale_embed rows (the T table needs them all), without it after the window rows (the first
  // barrier waits for those anyway).  Requested after every other load, they made wave 0 wait
  // for its long-range key gathers before the first barrier.
  const int jc = tid < J ? tid : J - 1;
  float bias_ld = 0.f, gain_ld = 1.f;
  SeRows<D> seR;
  if constexpr (HAS_SE) {
    bias_ld = p.pos_bias[jc * p.H + h];
    gain_ld = p.score_gain ? p.score_gain[h * J + jc] : 1.0f;
    seR.load(p.scale_embed, J, tid);
  }
  bf16x8_t qB[KS];
  if constexpr (HAS_SE) {
    const int qlane = opaque(i * qsn + 8 * g);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qB[s] = as_bf16x8(bload16(rQ, n0w * qsn + (8 * g + 32 * s < D ? qlane + 32 * s : kNoElem)));
  }
  uint4 qR[CHW];
#pragma unroll
  for (int u = 0; u < CHW; ++u) qR[u] = bload16(rQ, n0w * qsn + qlaneR[u]);
  // Offsets are (uniform row) * stride + (per-lane part), so the row products stay scalar.
  uint4 wv[CWIN], wk[CWIN];
#pragma unroll
  for (int u = 0; u < CWIN; ++u) {
    const int ci = tid + u * kBlock;
    const bool cv = ci % CPS < CPR;
    wv[u] = bload16(rV, (n0 - kMaxWindow) * vsn + opaque(cv ? (ci / CPS) * vsn + (ci % CPS) * 8 : kNoElem));
    wk[u] = bload16(rK, (n0 - kMaxWindow) * ksn + opaque(cv ? (ci / CPS) * ksn + (ci % CPS) * 8 : kNoElem));
  }
  if constexpr (!HAS_SE) {
    bias_ld = p.pos_bias[jc * p.H + h];
    gain_ld = p.score_gain ? p.score_gain[h * J + jc] : 1.0f;
  }
  // The long-range key rows n0w - delta + 0..15 in the row-chunk layout, in two groups (the
  // second after the dense band has consumed its registers) to bound the register peak; three
  // for D > 64, whose rows take three 16-byte pieces per lane where D = 64's take two (in two
  // groups they spill at three workgroups per CU).
  constexpr int NGRP = D > 64 ? 3 : 2;
  // Group boundaries: taps [0, NH), [NH, NH2), [NH2, NSM).  The first group, live with the window
  // rows, is the smallest.
  constexpr int NH = NGRP == 2 ? (NSM + 1) / 2 : (NSM + 3) / 4;
  constexpr int NH2 = NGRP == 2 ? NSM : NH + (NSM - NH + 1) / 2;
  uint4 kS[NSM][CHW];
#pragma unroll
  for (int t = 0; t < NH; ++t) {
    if (NSC > 0 || t < NS) {
      const int m0 = n0w - dl_s[t];
#pragma unroll
      for (int u = 0; u < CHW; ++u) kS[t][u] = bload16(rK, m0 * ksn + klaneR[u]);
    }
  }
  if (tid < J) {
    sBias2[tid] = bias_ld * kLog2e;
    sGain2[tid] = gain_ld * c2;
  }
  float* sTw = reinterpret_cast<float*>(sVs[w]);  // T table until the long-range P V
  if constexpr (HAS_SE) {
    // T[i][j] = log2e (bias_j + c q_i.se_j) for every tap, SE Q^T on the MFMA.  scale_embed is
    // staged as two bf16 planes, hi = bf16(se) in the K window and lo = bf16(se - hi) in the V
    // window (both still free: the window rows are in flight in registers), so q.se keeps se's
    // fp32 precision to about 2^-17.
    bf16_t* const sSE = sK;
    bf16_t* const sSElo = sV;
    seR.template store<RV>(sSE, sSElo, tid);
    __syncthreads();
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
        if (j < J) sTw[i * TS + j] = fmaf(c2, acc[r], sBias2[j]);
      }
    }
    __syncthreads();  // every wave has read the planes: the window rows move in
  }
#pragma unroll
  for (int u = 0; u < CWIN; ++u) {
    const int ci = tid + u * kBlock;
    const int r = ci / CPS, cc = ci - r * CPS;
    if (ci < WIN * CPS) {
      st16(sV + r * RV + cc * 8, wv[u]);
      st16(sK + r * RV + cc * 8, wk[u]);
    }
  }
  if constexpr (!HAS_SE) {
#pragma unroll
    for (int u = 0; u < CHW; ++u)
      if (rc_valid<D>(l, u)) st16(sVs[w] + rc_row<D>(l, u) * RV + rc_chunk<D>(l, u) * 8, qR[u]);
  }
  __syncthreads();
  if constexpr (!HAS_SE) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qB[s] = 8 * g + 32 * s < D ? as_bf16x8(*reinterpret_cast<const uint4*>(sVs[w] + i * RV + 8 * g + 32 * s))
                                 : as_bf16x8(zero16());
  }

  // ---- Dense band scores: S^T = K_band Q^T. ----
  f32x4_t accS[3];
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    accS[kk] = zero4();
    const bf16_t* kr = sK + (16 * w + 16 * kk + i) * RV + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      accS[kk] = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(kr + 32 * s)), qB[s], accS[kk]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Long-range q.k on the VALU: each lane dots its 16-byte chunks of a row, the row's lanes sum
  // (DPP), and one lane per row files the score in the wave's [query][tap] table.  The first
  // half's registers are free before the second half is loaded.
  float* sRw = reinterpret_cast<float*>(sVs[w]);  // (unused with scale_embed)
  // Score of long-range tap t for each of the wave's rows, less the bias and q.se term
  // (log2 units): gain c log2e q.k, one DPP sum per row.
  auto sparse_score = [&](int t) {
    const int j = W + 1 + t;
#pragma unroll
    for (int rg = 0; rg < CHW / CPL; ++rg) {
      float d = dot8_bf16(qR[rg * CPL], kS[t][rg * CPL], 0.f);
#pragma unroll
      for (int pc = 1; pc < CPL; ++pc) d += dot8_bf16(qR[rg * CPL + pc], kS[t][rg * CPL + pc], 0.f);
      d = group_sum<G_::CPRP>(sGain2[j] * d);
      if (l % G_::CPRP == 0) {
        if constexpr (HAS_SE) sTw[rc_row<D>(l, rg * CPL) * TS + j] += d;
        else sRw[rc_row<D>(l, rg * CPL) * TR + t] = d;
      }
    }
  };
#pragma unroll
  for (int t = 0; t < NH; ++t)
    if (NSC > 0 || t < NS) sparse_score(t);
  auto load_k = [&](int t0, int t1) {
#pragma unroll
    for (int t = t0; t < t1; ++t) {
      if (NSC > 0 || t < NS) {
        const int m0 = n0w - dl_s[t];
#pragma unroll
        for (int u = 0; u < CHW; ++u) kS[t][u] = bload16(rK, m0 * ksn + klaneR[u]);
      }
    }
  };
  load_k(NH, NH2);
  int vlane[CHW];  // this lane's chunks of a wave's 16-row V block (row-chunk layout)
#pragma unroll
  for (int u = 0; u < CHW; ++u) vlane[u] = opaque(rc_lane<D>(l, u, vsn));
  uint4 vS[PF][CHW];  // long-range V rows n0w - delta + 0..15, PF taps ahead
  auto prefetch_v = [&]() {
#pragma unroll
    for (int t = 0; t < PF; ++t) {
      if (t < NS) {
        const int r0 = n0w - dl_s[t];
#pragma unroll
        for (int u = 0; u < CHW; ++u) vS[t][u] = bload16(rV, r0 * vsn + vlane[u]);
      }
    }
  };
  // With three groups the V rows are requested after the last group is scored (their registers
  // are the last group's).
  if constexpr (NGRP == 2) prefetch_v();

  __builtin_amdgcn_sched_barrier(0);

  // Scores in log2 units: s2 = gain*c*log2e * q.k + log2e*(bias + c q.se).
  float sd[12];
  const int dl0 = 32 - 4 * g + i;
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dl = dl0 - 16 * kk - r;  // n - m for key m of this register
      const bool ok = row_ok && (unsigned)dl <= (unsigned)W && n >= dl;
      const int j = ok ? dl : 0;
      const float v = fmaf(sGain2[j], accS[kk][r], HAS_SE ? sTw[i * TS + j] : sBias2[j]);
      sd[kk * 4 + r] = ok ? v : -INFINITY;
    }
  }

#pragma unroll
  for (int t = NH; t < NH2; ++t)
    if (NSC > 0 || t < NS) sparse_score(t);
  if constexpr (NGRP == 3) {
    __builtin_amdgcn_sched_barrier(0);
    load_k(NH2, NSM);
#pragma unroll
    for (int t = NH2; t < NSM; ++t)
      if (NSC > 0 || t < NS) sparse_score(t);
    __builtin_amdgcn_sched_barrier(0);
    prefetch_v();
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the table is written
  __builtin_amdgcn_wave_barrier();
  // The diagonal lane of query i (group i/4, register i%4) owns its long-range taps: the
  // one-hot P operand of the long-range P V below must sit there.
  const bool diag = g == (i >> 2);
  float ss[NSM];
#pragma unroll
  for (int t = 0; t < NSM; ++t) {
    ss[t] = -INFINITY;
    if (NSC > 0 || t < NS) {
      const int j = W + 1 + t;
      const float v = HAS_SE ? sTw[i * TS + j] : sRw[i * TR + t] + sBias2[j];
      ss[t] = (diag && row_ok && n >= dl_s[t]) ? v : -INFINITY;
    }
  }

  // ---- Softmax over the J taps of each query column (base 2). ----
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < 12; ++e) mx = fmaxf(mx, sd[e]);
#pragma unroll
  for (int t = 0; t < NSM; ++t) mx = fmaxf(mx, ss[t]);
  mx = col_max(mx);
  if (mx == -INFINITY) mx = 0.f;  // row past N
  float lsum = 0.f;
#pragma unroll
  for (int e = 0; e < 12; ++e) { sd[e] = __builtin_amdgcn_exp2f(sd[e] - mx); lsum += sd[e]; }
#pragma unroll
  for (int t = 0; t < NSM; ++t) { ss[t] = __builtin_amdgcn_exp2f(ss[t] - mx); lsum += ss[t]; }
  lsum = col_sum(lsum);
  const long long rowbase = ((long long)b * p.H + h) * N;
  if (row_ok && g == 0 && p.lse) p.lse[rowbase + n] = (mx + __log2f(lsum)) * 0.6931471805599453f;
  const float inv = row_ok ? if_a / lsum : 0.f;
  // The long-range taps' weights alpha_j = e_j / sum (zero where masked) for the backward, which
  // then recomputes no long-range score: [b,h][tap][query], written by the query's diagonal lane.
  if (p.alpha_lr && diag && row_ok) {
    float* const alw = p.alpha_lr + ((long long)(b * p.H + h) * NS) * N + n;
    const float rl = 1.0f / lsum;
#pragma unroll
    for (int t = 0; t < NSM; ++t)
      if (NSC > 0 || t < NS) alw[(long long)t * N] = ss[t] * rl;
  }

  // ---- Dense P V: O^T = V^T P^T. ----
  f32x4_t accO[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) accO[db] = zero4();
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    const s16x4_t pb = pack_bf16x4(sd[4 * kk] * inv, sd[4 * kk + 1] * inv, sd[4 * kk + 2] * inv,
                                   sd[4 * kk + 3] * inv);
    const bf16_t* vr = sV + (16 * w + 16 * kk + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
    for (int db = 0; db < DB; ++db) accO[db] = mfma_16x16x16(lds_read_tr16(vr + 16 * db), pb, accO[db]);
  }

  // ---- Long-range P V on the MFMA: O^T += V_t^T P_t^T per tap. ----
  // The tap's 16 V rows (gathered whole-row) are staged in the wave's block in natural row order
  // and read back transposed (ds_read_tr16_b64) as the A operand; P_t^T is one-hot: only the
  // diagonal lane of query i holds a weight (the others' ss[t] are exp2(-inf) = 0), at key i.
  bf16_t* const sSt = sVs[w];
  const bf16_t* const vtr = sSt + (4 * g + (i >> 2)) * RV + 4 * (i & 3);
  const uint2 ohm = onehot_masks(i & 3);
#pragma unroll
  for (int t = 0; t < NSM; ++t) {
    if (NSC > 0 || t < NS) {
#pragma unroll
      for (int u = 0; u < CHW; ++u)
        if (rc_valid<D>(l, u)) st16(sSt + rc_row<D>(l, u) * RV + rc_chunk<D>(l, u) * 8, vS[t % PF][u]);
      if (t + PF < NS) {
        const int r0 = n0w - dl_s[t + PF];
#pragma unroll
        for (int u = 0; u < CHW; ++u) vS[t % PF][u] = bload16(rV, r0 * vsn + vlane[u]);
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the rows are staged
      __builtin_amdgcn_wave_barrier();
      // The weight rounded to bf16, as the dense band's P V rounds its weights.
      const s16x4_t pb = onehot_bf16x4(ss[t] * inv, ohm);
#pragma unroll
      for (int db = 0; db < DB; ++db) accO[db] = mfma_16x16x16(lds_read_tr16(vtr + 16 * db), pb, accO[db]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- out (MFMA layout: lane (i, g) holds query i, d = 16 db + 4 g + 0..3) leaves as whole
  // rows: the lanes deposit bf16 quads in the wave's block, then 16-byte row pieces are stored.
  bf16_t* outb = static_cast<bf16_t*>(p.out) + b * p.os.b + h * p.os.h;
#pragma unroll
  for (int db = 0; db < DB; ++db)
    *reinterpret_cast<uint2*>(sSt + i * RV + 16 * db + 4 * g) =
        pack_bf16x4_u2(accO[db][0], accO[db][1], accO[db][2], accO[db][3]);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    const int rr = rc_row<D>(l, u), cc = rc_chunk<D>(l, u);
    if (n0w + rr < N && cc < CPR)
      st16(outb + (n0w + rr) * p.os.n + 8 * cc, *reinterpret_cast<const uint4*>(sSt + rr * RV + 8 * cc));
  }
}

template <int D, bool HAS_SE>
static void launch_fwd_mfma_ns(const FwdParams& p, unsigned nblocks, hipStream_t st) {
  // Long-range tap counts of the named tables (44, 46, 47 offsets) get fully unrolled kernels.
  switch (p.taps.J - p.taps.W - 1) {
    case 11: hipLaunchKernelGGL((fwd_mfma_kernel<D, HAS_SE, 11>), dim3(nblocks), dim3(kBlock), 0, st, p); break;
    case 13: hipLaunchKernelGGL((fwd_mfma_kernel<D, HAS_SE, 13>), dim3(nblocks), dim3(kBlock), 0, st, p); break;
    case 14: hipLaunchKernelGGL((fwd_mfma_kernel<D, HAS_SE, 14>), dim3(nblocks), dim3(kBlock), 0, st, p); break;
    default: hipLaunchKernelGGL((fwd_mfma_kernel<D, HAS_SE, 0>), dim3(nblocks), dim3(kBlock), 0, st, p); break;
  }
}

template <int D>
static hipError_t launch_fwd_mfma_d(const FwdParams& p0, hipStream_t st) {
  FwdParams p = p0;
  p.n_tiles = (p.N + 63) / 64;
  const long long nblocks = (long long)p.B * p.H * p.n_tiles;
  if (nblocks == 0) return hipSuccess;
  if (p.scale_embed) launch_fwd_mfma_ns<D, true>(p, (unsigned)nblocks, st);
  else launch_fwd_mfma_ns<D, false>(p, (unsigned)nblocks, st);
  return hipGetLastError();
}

bool fwd_mfma_supported(const FwdParams& p, int D) {
  // Buffer offsets are 32-bit: every row a tap can touch must stay below 2^31 bytes.
  const long long rs = p.qs.n > p.ks.n ? (p.qs.n > p.vs.n ? p.qs.n : p.vs.n)
                                        : (p.ks.n > p.vs.n ? p.ks.n : p.vs.n);
  const long long rmin = p.qs.n < p.ks.n ? (p.qs.n < p.vs.n ? p.qs.n : p.vs.n)
                                          : (p.ks.n < p.vs.n ? p.ks.n : p.vs.n);
  const long long span = ((long long)p.N + p.taps.maxd + 64) * rs * 2;
  return (D == 32 || D == 64 || D == 80 || D == 96 || D == 128) && p.taps.J - p.taps.W - 1 <= kMaxSparse &&
         rmin >= D && span < (1LL << 31);
}

hipError_t launch_fwd_mfma(const FwdParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return launch_fwd_mfma_d<32>(p, st);
    case 64: return launch_fwd_mfma_d<64>(p, st);
    case 80: return launch_fwd_mfma_d<80>(p, st);
    case 96: return launch_fwd_mfma_d<96>(p, st);
    case 128: return launch_fwd_mfma_d<128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsqg
