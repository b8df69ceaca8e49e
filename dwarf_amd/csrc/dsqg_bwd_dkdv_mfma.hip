// DSQG backward, launch 2, bf16 MFMA path (gfx950): key-centric dk and dv.
//
// A workgroup owns one (b,h) and 64 key rows [m0, m0+64); wave w owns keys m0w = m0+16w .. +15.
// Key m is read by the queries n = m + delta_j, so
//   dv_m = sum_j a alpha_j(n) dOut_n,      dk_m = sum_j c g_j dS_j(n) q_n,
//   alpha_j(n) = exp(s_j(n) - lse_n),      dS_j(n) = a alpha_j(n) (dOut_n . v_m - D'_n),
// with lse from the forward and D' from launch 1.
//  * Dense band: the wave's keys meet queries [m0w, m0w+48) in three 16x16 tiles
//    S = Q K^T and U = dOut V^T (A = query rows, B = the wave's key / value rows).  In the MFMA
//    result layout lane l holds key column l%16 and query rows 4*(l/16)+r, which is exactly the
//    B operand of dK^T = Q^T (c g dS) and dV^T = dOut^T (a alpha); Q^T and dOut^T come from the
//    query window [m0, m0+96) in LDS through ds_read_tr16_b64.
//  * Long-range taps: query rows m0w + delta + 0..15, loaded in the row-chunk layout (each
//    group of four lanes reads 64 contiguous bytes of a row: the vector L1 serves that at close
//    to four times the rate of the MFMA operand order; at D = 96 every lane carries three
//    chunks of one row, none idle).  Their
//    weights come from launch 1, which has every long-range pair's alpha, u and D' in hand
//    anyway: per (query, tap) the pair (c g_j dS_j, a alpha_j) as two bf16 in one dword, so
//    this launch computes no long-range score and reads no long-range lse or D'.  A tap adds a
//    scaled query / dOut row to each key's row (no contraction), so it runs on the VALU in the
//    row layout (v_dot2_f32_bf16 against (w, 0) / (0, w)), after the band's accumulators are
//    turned into that layout once; no LDS traffic per tap.  (Each of these 11 of the 44 terms
//    of dk and dv carries the 2^-9 relative rounding of one bf16 weight; the band's 33 keep
//    fp32 weights as hi + lo pairs.)  The LDS fits four workgroups per CU up to D = 96 (three
//    with scale_embed above D = 64).
//  * The dense band's weights enter their MFMAs as bf16 hi + lo pairs (two products each).
//  * The q.se_j term of the band's scores (scale_embed) is a [query][tap] table per wave computed
//    on the MFMA (Q SE^T) with se rounded to bf16 (an error of about 2^-9 |c q.se| in the score,
//    1e-4 at the reference's se ~ 0.05; the parameter gradients come from launch 1, which keeps
//    se at fp32 precision).
// With p.red_blocks > 0 the launch carries that many extra workgroups at the end of the grid,
// which sum the parameter-gradient partials (dsqg_reduce.hpp) while the dk/dv tiles run.
// Follows _bwd_dkdv_v3 (kernels/dsqg_attention_v3.py:282-352).
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_mfma.hpp"
#include "dsqg_reduce.hpp"

namespace dsqg {

// Occupancy targets: four workgroups per CU (at most 128 VGPRs and 40 KB of LDS each) up to
// D = 96; three for the scale_embed forms above D = 64, whose se rows and T table take 52 KB of
// LDS; none at D = 128 (its registers and LDS set it).
template <int D, bool HAS_SE, int NSC>
__global__ __launch_bounds__(kBlock, D == 128 ? 1 : (D > 64 && HAS_SE ? 3 : 4)) void bwd_dkdv_mfma_kernel(BwdParams p) {
  using G_ = Geo<D>;
  constexpr int KT = 64;                  // key rows per workgroup
  constexpr int KS = G_::KS;
  constexpr int DB = G_::DB;
  constexpr int RV = G_::RV;              // LDS row stride (36 dwords at D=64)
  constexpr int WIN = KT + kMaxWindow;    // query window rows [m0, m0+96)
  constexpr int CPR = G_::CPR;
  constexpr int CPS = G_::CPS;            // chunks per staged (padded) row
  constexpr int CWIN = (WIN * CPS + kBlock - 1) / kBlock;
  constexpr int CHW = G_::CHW;            // 16-byte chunks per lane of a wave's 16-row block
  constexpr int NSM = NSC > 0 ? NSC : kMaxSparse;
  // Long-range taps in flight: a tap is a few dozen VALU instructions per wave, so the loads
  // run several taps ahead (as many as the register budget of the occupancy target allows).
  constexpr int PF = D > 64 ? 2 : ((D == 64 && !HAS_SE) ? 3 : 4);
  // [query][dense tap] table, row stride 33 (the dense taps): the band's diagonal reads (row
  // 4g + r, tap 4g + r - i) meet at most two to a bank, as with any stride of 33..35, and the
  // table stays small enough for four workgroups per CU.
  constexpr int TS = 33;
  constexpr int SEJ = 48;
  constexpr float kLog2e = 1.4426950408889634f;

  // Query window, then dOut window (one array: after the band each wave takes a quarter of it
  // to turn its accumulators into row layout).  With scale_embed the se rows sit in the dOut
  // window until the T table is built, and the dOut rows are stored after it: the workgroup's LDS
  // then fits four workgroups per CU (40 KB each at D = 64).
  __shared__ __align__(16) bf16_t sQO[2 * WIN * RV];
  bf16_t* const sQ = sQO;
  bf16_t* const sO = sQO + WIN * RV;
  static_assert(SEJ <= WIN, "the se rows fit the dOut window");
  bf16_t* const sSE = sO;
  __shared__ float sT[HAS_SE ? WIN * TS : 1];        // log2e (bias + c q.se), window query x dense tap
  auto t_at = [&](int row, int j) { return row * TS + j; };
  __shared__ float sBias2[kMaxTaps];
  __shared__ float sGain2[kMaxTaps];                 // gain * c * log2e
  __shared__ float sGainC[HAS_SE ? 1 : kMaxTaps];    // gain * c (with scale_embed: sGain2 ln 2)

  const int tid = threadIdx.x;
  // Workgroups past the dk/dv tiles run the parameter reduction (partials from launch 1).
  const int kv_blocks = (int)gridDim.x - p.red_blocks;
  if ((int)blockIdx.x >= kv_blocks) {
    reduce_params_wave(p.red, ((int)blockIdx.x - kv_blocks) * (kBlock / 64) + __builtin_amdgcn_readfirstlane(tid >> 6), tid & 63);
    return;
  }
  // The kernel arguments of the prologue in one round trip: sizes and input strides pass through
  // an empty asm statement that the code after it depends on, the input pointers are its
  // operands, so all are requested before it and waited for once (otherwise the grid constants
  // come first, the block-number divisions wait for them, and each later group of arguments
  // costs another dependent round trip).
  asm volatile("" : "+s"(p.H), "+s"(p.N), "+s"(p.n_tiles_kv), "+s"(p.taps.J), "+s"(p.taps.W),
               "+s"(p.qs.b), "+s"(p.qs.h), "+s"(p.qs.n), "+s"(p.ks.b), "+s"(p.ks.h), "+s"(p.ks.n),
               "+s"(p.vs.b), "+s"(p.vs.h), "+s"(p.vs.n), "+s"(p.dos.b), "+s"(p.dos.h), "+s"(p.dos.n)
               : "s"(p.q), "s"(p.k), "s"(p.v), "s"(p.dout), "s"(p.lse), "s"(p.dpre), "s"(p.pos_bias),
                 "s"(p.if_gain));
  const int lb = xcd_logical_block(blockIdx.x, kv_blocks);
  const int bh = lb / p.n_tiles_kv, tile = lb - bh * p.n_tiles_kv;
  const int b = bh / p.H, h = bh - b * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const int NS = NSC > 0 ? NSC : J - W - 1;
  const float c = p.scale, c2 = p.scale * kLog2e;
  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const int qsn = (int)p.qs.n, ksn = (int)p.ks.n, vsn = (int)p.vs.n, dosn = (int)p.dos.n;
  const int m0 = tile * KT;
  const long long rowbase = ((long long)b * p.H + h) * N;

  const __amdgpu_buffer_rsrc_t rQ = slice_rsrc(static_cast<const bf16_t*>(p.q) + b * p.qs.b + h * p.qs.h, p.qs.n, N, D);
  const __amdgpu_buffer_rsrc_t rK = slice_rsrc(static_cast<const bf16_t*>(p.k) + b * p.ks.b + h * p.ks.h, p.ks.n, N, D);
  const __amdgpu_buffer_rsrc_t rV = slice_rsrc(static_cast<const bf16_t*>(p.v) + b * p.vs.b + h * p.vs.h, p.vs.n, N, D);
  const __amdgpu_buffer_rsrc_t rO = slice_rsrc(static_cast<const bf16_t*>(p.dout) + b * p.dos.b + h * p.dos.h, p.dos.n, N, D);
  const __amdgpu_buffer_rsrc_t rL = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.lse + rowbase), (short)0, N * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rP = __builtin_amdgcn_make_buffer_rsrc(p.dpre + rowbase, (short)0, N * 4, 0x00020000);

  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, i = l & 15, g = l >> 4;
  const int m0w = m0 + 16 * w;
  const int m = m0w + i;                  // key row of this lane's MFMA column
  const bool key_ok = m < N;
  int dl_s[NSM];
  load_sparse_deltas(p.taps, dl_s);
  const int klane = opaque(i * ksn + 8 * g), vlane = opaque(i * vsn + 8 * g);
  // Row-chunk layout for the long-range query / dOut rows.
  int qlaneR[CHW], olaneR[CHW];
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    qlaneR[u] = opaque(rc_lane<D>(l, u, qsn));
    olaneR[u] = opaque(rc_lane<D>(l, u, dosn));
  }

  // ---- Loads (scale_embed first: the T table waits for it alone). ----
  SeRows<D> seR;
  if constexpr (HAS_SE) seR.load(p.scale_embed, J, tid);
  uint4 wq[CWIN], wo[CWIN];
#pragma unroll
  for (int u = 0; u < CWIN; ++u) {
    const int ci = tid + u * kBlock;
    const bool cv = ci % CPS < CPR;
    wq[u] = bload16(rQ, m0 * qsn + opaque(cv ? (ci / CPS) * qsn + (ci % CPS) * 8 : kNoElem));
    wo[u] = bload16(rO, m0 * dosn + opaque(cv ? (ci / CPS) * dosn + (ci % CPS) * 8 : kNoElem));
  }
  // Per-tap bias and gain (J <= kMaxTaps < kBlock: one per thread), requested with the window
  // rows, so that storing them below waits for those rows only (requested after every load,
  // they made wave 0 wait for all of its loads before the first barrier).
  const int jc = tid < J ? tid : J - 1;
  const float bias_ld = p.pos_bias[jc * p.H + h];
  const float gain_ld = p.score_gain ? p.score_gain[h * J + jc] : 1.0f;
  bf16x8_t kB[KS], vB[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const bool sv = 8 * g + 32 * s < D;  // the zero columns of D = 80's last K-step
    kB[s] = as_bf16x8(bload16(rK, m0w * ksn + (sv ? klane + 32 * s : kNoElem)));
    vB[s] = as_bf16x8(bload16(rV, m0w * vsn + (sv ? vlane + 32 * s : kNoElem)));
  }
  // lse (log2 units) and D' of the band's queries m0w + 16qb + 4g + r.
  float lq[12], dq_[12];
#pragma unroll
  for (int qb = 0; qb < 3; ++qb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nq = m0w + 16 * qb + 4 * g + r;
      lq[4 * qb + r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rL, (unsigned)(nq * 4), 0, 0)) * kLog2e;
      dq_[4 * qb + r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rP, (unsigned)(nq * 4), 0, 0));
    }
  // Weights of the long-range taps from launch 1: each lane reads the dword of the query that its
  // row-layout rows meet (key row m0w + r, query m0w + r + delta), PF taps ahead like the query
  // rows.  One buffer resource per tap over the [N] dwords of the (b,h) and tap, so a query at or
  // past N reads as a zero weight.
  const unsigned* const lwb = reinterpret_cast<const unsigned*>(p.lrw) + (long long)bh * NS * N;
  unsigned wS[PF][CHW];
  auto load_w = [&](int t) {
    const __amdgpu_buffer_rsrc_t rW =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned*>(lwb + (long long)t * N), (short)0, N * 4, 0x00020000);
#pragma unroll
    for (int u = 0; u < CHW; ++u)
      wS[t % PF][u] = __builtin_amdgcn_raw_buffer_load_b32(rW, (unsigned)(m0w + rc_row<D>(l, u) + dl_s[t]) * 4u, 0, 0);
  };

  if (tid < J) {
    sBias2[tid] = bias_ld * kLog2e;
    sGain2[tid] = gain_ld * c2;
    if constexpr (!HAS_SE) sGainC[tid] = gain_ld * c;
  }
  if constexpr (HAS_SE) seR.template store<RV>(sSE, nullptr, tid);
  auto store_window = [&](bf16_t* dst, const uint4 (&src)[CWIN]) {
#pragma unroll
    for (int u = 0; u < CWIN; ++u) {
      const int ci = tid + u * kBlock;
      if (ci < WIN * CPS) st16(dst + (ci / CPS) * RV + (ci % CPS) * 8, src[u]);
    }
  };
  store_window(sQ, wq);
  if constexpr (!HAS_SE) store_window(sO, wo);
  __syncthreads();

  if constexpr (HAS_SE) {
    // T[row][j] = log2e (bias_j + c q.se_j) for the 96 window queries (Q SE^T) and the dense
    // taps j <= W, 16-row blocks w and w+4 per wave (before the band's accumulators are live).
    for (int blk = w; blk < WIN / 16; blk += 4) {
      const bf16_t* qr = sQ + (16 * blk + i) * RV + 8 * g;
#pragma unroll
      for (int jb = 0; jb < 3; ++jb) {
        f32x4_t acc = zero4();
        const bf16_t* sr = sSE + (16 * jb + i) * RV + 8 * g;
#pragma unroll
        for (int s = 0; s < KS; ++s)
          acc = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(qr + 32 * s)),
                              as_bf16x8(*reinterpret_cast<const uint4*>(sr + 32 * s)), acc);
        const int j = 16 * jb + i;  // column = tap, rows = queries 4g + r
        if (j <= W) {
#pragma unroll
          for (int r = 0; r < 4; ++r) sT[t_at(16 * blk + 4 * g + r, j)] = fmaf(c2, acc[r], sBias2[j]);
        }
      }
    }
    __syncthreads();  // every wave has read the se rows: the dOut rows move in
    store_window(sO, wo);
    __syncthreads();
  }

  // ---- Dense band: S = Q K^T, U = dOut V^T for query blocks qb = 0..2. ----
  f32x4_t accS[3], accU[3];
#pragma unroll
  for (int qb = 0; qb < 3; ++qb) {
    accS[qb] = zero4();
    accU[qb] = zero4();
    const bf16_t* qr = sQ + (16 * w + 16 * qb + i) * RV + 8 * g;
    const bf16_t* orr = sO + (16 * w + 16 * qb + i) * RV + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      accS[qb] = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(qr + 32 * s)), kB[s], accS[qb]);
      accU[qb] = mfma_16x16x32(as_bf16x8(*reinterpret_cast<const uint4*>(orr + 32 * s)), vB[s], accU[qb]);
    }
  }
  f32x4_t dK[DB], dV[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) { dK[db] = zero4(); dV[db] = zero4(); }
#pragma unroll
  for (int qb = 0; qb < 3; ++qb) {
    float wk[4], wv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dl = 16 * qb + 4 * g + r - i;  // query - key
      const int nq = m0w + 16 * qb + 4 * g + r;
      const bool ok = key_ok && (unsigned)dl <= (unsigned)W && nq < N;
      const int j = ok ? dl : 0;
      const float s2 = fmaf(sGain2[j], accS[qb][r],
                            HAS_SE ? sT[t_at(16 * w + 16 * qb + 4 * g + r, j)] : sBias2[j]);
      const float alpha = ok ? __builtin_amdgcn_exp2f(s2 - lq[4 * qb + r]) : 0.f;
      const float dS = a * alpha * (accU[qb][r] - dq_[4 * qb + r]);
      wk[r] = (HAS_SE ? sGain2[j] * 0.6931471805599453f : sGainC[j]) * dS;
      wv[r] = a * alpha;
    }
    // The weights as bf16 hi + lo pairs, so the products keep their fp32 precision.
    s16x4_t bk, bkl, bv, bvl;
    split_bf16x4(wk[0], wk[1], wk[2], wk[3], bk, bkl);
    split_bf16x4(wv[0], wv[1], wv[2], wv[3], bv, bvl);
    const bf16_t* qr = sQ + (16 * w + 16 * qb + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
    const bf16_t* orr = sO + (16 * w + 16 * qb + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const s16x4_t qt = lds_read_tr16(qr + 16 * db), ot = lds_read_tr16(orr + 16 * db);
      dK[db] = mfma_16x16x16(qt, bk, dK[db]);
      dK[db] = mfma_16x16x16(qt, bkl, dK[db]);
      dV[db] = mfma_16x16x16(ot, bv, dV[db]);
      dV[db] = mfma_16x16x16(ot, bvl, dV[db]);
    }
  }

  // ---- Long-range taps: queries m0w + delta + 0..15, one per key row. ----
  // Each tap adds a scaled query / dOut row to each key's dk / dv row (dk_m += c g_j dS q_n,
  // dv_m += a alpha_j dOut_n with n = m + delta_j): no contraction, so it runs on the VALU in
  // the row-chunk layout the gathered rows arrive in (8 elements per lane and chunk), as
  // v_dot2_f32_bf16 against (w, 0) and (0, w) (exact products of the bf16 row and bf16 weight,
  // fp32 sums), with no LDS staging and no wait per tap.  The band's MFMA accumulators are first
  // turned into that layout through the wave's share of the (now free) window tiles.
  // Their first loads are issued only now: during the band the registers hold the band's
  // operands, and four workgroups per CU cover the wait.  Scheduling barriers keep every tap's
  // loads where they stand (the scheduler otherwise hoists later taps' loads over the
  // conversion and the earlier taps' sums, and their registers spill).
  uint4 qS[PF][CHW], oS[PF][CHW];
  auto load_tap = [&](int t) {
    load_w(t);
    const int n0 = m0w + dl_s[t];
#pragma unroll
    for (int u = 0; u < CHW; ++u) {
      qS[t % PF][u] = bload16(rQ, n0 * qsn + qlaneR[u]);
      oS[t % PF][u] = bload16(rO, n0 * dosn + olaneR[u]);
    }
  };
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < PF; ++t)
    if (t < NS) load_tap(t);
  __builtin_amdgcn_sched_barrier(0);

  // MFMA layout (lane (i, g): key i, d = 16 db + 4 g + 0..3) -> row-chunk layout (lane: key
  // row rc_row, d = 8 rc_chunk + 0..7), fp32, one matrix at a time through the wave's quarter
  // of the window tiles (row stride DP + 4 floats: conflict-free 16-byte writes).
  constexpr int CS = G_::DP + 4;
  static_assert(16 * CS * 4 <= 2 * WIN * RV * 2 / 4, "row-layout staging fits a quarter of the window tiles");
  float* const cvt = reinterpret_cast<float*>(sQO) + w * (2 * WIN * RV / 2 / 4);
  float kacc[CHW][8], vacc[CHW][8];
  __syncthreads();  // every wave's band reads of sQ / sO are done
  auto to_rows = [&](const f32x4_t (&acc)[DB], float (&dst)[CHW][8]) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
      *reinterpret_cast<float4*>(cvt + i * CS + 16 * db + 4 * g) = make_float4(acc[db][0], acc[db][1], acc[db][2], acc[db][3]);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the quads are written
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int u = 0; u < CHW; ++u) {
      const bool ok = rc_valid<D>(l, u);
      const float* src = cvt + (ok ? rc_row<D>(l, u) * CS + 8 * rc_chunk<D>(l, u) : 0);
      const float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
      dst[u][0] = ok ? lo.x : 0.f; dst[u][1] = ok ? lo.y : 0.f; dst[u][2] = ok ? lo.z : 0.f; dst[u][3] = ok ? lo.w : 0.f;
      dst[u][4] = ok ? hi.x : 0.f; dst[u][5] = ok ? hi.y : 0.f; dst[u][6] = ok ? hi.z : 0.f; dst[u][7] = ok ? hi.w : 0.f;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the rows are read before the next matrix
    __builtin_amdgcn_wave_barrier();
  };
  to_rows(dK, kacc);
  to_rows(dV, vacc);
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int t = 0; t < NSM; ++t) {
    if (NSC > 0 || t < NS) {
      const int slot = t % PF;
#pragma unroll
      for (int u = 0; u < CHW; ++u) {
        // This row's weights: bf16 dk weight in the low half, bf16 dv weight in the high half.
        const unsigned wt = wS[slot][u];
        const unsigned wk0 = wt & 0xffffu, wk1 = wt << 16, wv0 = wt >> 16, wv1 = wt & 0xffff0000u;
        const uint4 qv = qS[slot][u], ov = oS[slot][u];
        const unsigned qw[4] = {qv.x, qv.y, qv.z, qv.w}, ow[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kacc[u][2 * e] = dot2_bf16_bits(qw[e], wk0, kacc[u][2 * e]);
          kacc[u][2 * e + 1] = dot2_bf16_bits(qw[e], wk1, kacc[u][2 * e + 1]);
          vacc[u][2 * e] = dot2_bf16_bits(ow[e], wv0, vacc[u][2 * e]);
          vacc[u][2 * e + 1] = dot2_bf16_bits(ow[e], wv1, vacc[u][2 * e + 1]);
        }
      }
      // The tap's sums are due here (the empty asm pins them: the sums are pure arithmetic, which
      // instruction selection otherwise sinks past every later tap's loads to the stores).
#pragma unroll
      for (int u = 0; u < CHW; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(kacc[u][e]), "+v"(vacc[u][e]));
      __builtin_amdgcn_sched_barrier(0);
      if (t + PF < NS) load_tap(t + PF);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // dk, dv leave as whole rows straight from the row layout: 16-byte pieces per lane.
  {
    bf16_t* dkb = static_cast<bf16_t*>(p.dk) + b * p.dks.b + h * p.dks.h;
    bf16_t* dvb = static_cast<bf16_t*>(p.dv) + b * p.dvs.b + h * p.dvs.h;
#pragma unroll
    for (int u = 0; u < CHW; ++u) {
      const int rr = rc_row<D>(l, u), cc = rc_chunk<D>(l, u);
      if (rc_valid<D>(l, u) && m0w + rr < N) {
        uint4 kp, vp;
        kp.x = cvt_pk_bf16(kacc[u][0], kacc[u][1]); kp.y = cvt_pk_bf16(kacc[u][2], kacc[u][3]);
        kp.z = cvt_pk_bf16(kacc[u][4], kacc[u][5]); kp.w = cvt_pk_bf16(kacc[u][6], kacc[u][7]);
        vp.x = cvt_pk_bf16(vacc[u][0], vacc[u][1]); vp.y = cvt_pk_bf16(vacc[u][2], vacc[u][3]);
        vp.z = cvt_pk_bf16(vacc[u][4], vacc[u][5]); vp.w = cvt_pk_bf16(vacc[u][6], vacc[u][7]);
        st16(dkb + (m0w + rr) * p.dks.n + 8 * cc, kp);
        st16(dvb + (m0w + rr) * p.dvs.n + 8 * cc, vp);
      }
    }
  }
}

template <int D, bool HAS_SE>
static void launch_dkdv_mfma_ns(const BwdParams& p, unsigned nb, hipStream_t st) {
  switch (p.taps.J - p.taps.W - 1) {
    case 11: hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<D, HAS_SE, 11>), dim3(nb), dim3(kBlock), 0, st, p); break;
    case 13: hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<D, HAS_SE, 13>), dim3(nb), dim3(kBlock), 0, st, p); break;
    case 14: hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<D, HAS_SE, 14>), dim3(nb), dim3(kBlock), 0, st, p); break;
    default: hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<D, HAS_SE, 0>), dim3(nb), dim3(kBlock), 0, st, p); break;
  }
}

template <int D>
static hipError_t launch_dkdv_mfma_d(const BwdParams& p, unsigned nb, hipStream_t st) {
  if (p.scale_embed) launch_dkdv_mfma_ns<D, true>(p, nb, st);
  else launch_dkdv_mfma_ns<D, false>(p, nb, st);
  return hipGetLastError();
}

hipError_t launch_bwd_dkdv_mfma(const BwdParams& p, int D, unsigned nblocks, hipStream_t st) {
  switch (D) {
    case 32: return launch_dkdv_mfma_d<32>(p, nblocks, st);
    case 64: return launch_dkdv_mfma_d<64>(p, nblocks, st);
    case 80: return launch_dkdv_mfma_d<80>(p, nblocks, st);
    case 96: return launch_dkdv_mfma_d<96>(p, nblocks, st);
    case 128: return launch_dkdv_mfma_d<128>(p, nblocks, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace dsqg
