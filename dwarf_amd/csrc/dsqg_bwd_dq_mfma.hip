// DSQG backward, launch 1, bf16 MFMA path (gfx950): query-centric dq, D', the long-range taps'
// dk/dv weights and the per-workgroup parameter-gradient partials.
//
// A workgroup owns one (b,h) and 64 query rows [n0, n0+64); wave w owns rows n0w = n0+16w .. +15.
// With lse from the forward, every weight alpha_j = exp(s_j - lse) is known as soon as its
// score is, and the forward also stored the long-range taps' weights (alpha_lr), so:
//  1. Dense band (delta = 0..W): keys [n0w-32, n0w+16) as three 16x16 tiles, S^T = K Q^T and
//     U^T = V dOut^T on the MFMA (v_mfma_f32_16x16x32_bf16), alpha_j from S and lse, u_j = U.
//  2. Long-range pass 1, V rows only: u_j = dOut . v_j for tap j's 16 value rows n0w - delta + 0..15,
//     gathered in the row-chunk layout (64 contiguous bytes per 4 lanes) and dotted on the VALU
//     (v_dot2_f32_bf16, DPP sums over the row's lanes); each row's u goes to the wave's
//     [query][tap] table in LDS without a wait per tap.  Then D' = sum_j alpha_j u_j
//     (= dOut . o, pre-gain o) is exact (fp32 weights).
//  3. With D' known, dS_j = a alpha_j (u_j - D') and dq = c sum_j dS_j (g_j k_j + se_j):
//     the band's part as MFMAs K^T (c g dS)^T with K^T from LDS (ds_read_tr16_b64), whose weights
//     enter as bf16 hi + lo pairs, so the products keep fp32 weights, as the reference's fp32
//     sums do (kernels/dsqg_attention_v3.py:257-271).  The accumulators then turn into the row
//     layout once, and long-range pass 2, K rows only, adds each tap's scaled key row to each
//     query's row (no contraction) with fp32 FMAs on the VALU: exact bf16 keys, fp32 weights,
//     no LDS staging per tap.
//  4. dS fills the per-wave [query][tap] table, from which the workgroup sums dbias (and dg, da)
//     in a fixed order and dse = c sum_q dS q runs on the MFMA (Q^T dS over the tile's 64 queries,
//     its [D x J] output tiles split over the four waves).  Every long-range pair's dk/dv weights,
//     bf16(c g_j dS_j) and bf16(a alpha_j), go to the workspace ([b,h][tap][query] dwords) for
//     launch 2, so the key-centric pass needs no long-range score, lse or D' of its own.
// With scale_embed the band's q.se_j term is an MFMA (SE Q^T) filed in a per-wave [query][tap]
// table; se is staged as two bf16 planes (hi = bf16(se), lo = bf16(se - hi)) and dS in SE^T dS^T
// and in dse is split the same way, so these products carry se and dS at fp32 precision.
// The long-range taps' scores are not recomputed: their alpha comes from the forward.  With the
// score gain's gradient requested, c q.k of every pair is also needed: the band's from S, the
// long-range taps' from a dot product with the gathered key rows in pass 2.
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
__global__ __launch_bounds__(kBlock, D == 128 ? 1 : (D > 64 || (HAS_SE && NSC != 11) ? 2 : (HAS_SE || DG ? 3 : 4)))
void bwd_dq_mfma_kernel(BwdParams p) {
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
  constexpr int CPL = G_::CPL;            // chunks per lane and row
  constexpr int NSM = NSC > 0 ? NSC : kMaxSparse;
  // Long-range row blocks loaded ahead of use: as many as the register budget of the occupancy
  // target holds without spills (a tap is a few dozen VALU instructions per wave).  Four in the
  // plain 11-tap form; two above D = 64, in the scale_embed forms other than the 11-tap one
  // without the gain's gradient, and in the plain generic-table form; three otherwise.
  constexpr int PF = (D > 64 || (HAS_SE && (NSC != 11 || DG)) || (NSC == 0 && !DG))
                         ? 2
                         : (HAS_SE || DG || NSC != 11 ? 3 : 4);
  constexpr int TS = kDqTableStride;
  constexpr int TST = 38;                 // row stride of the dense-tap T table (2-way bank reads)
  constexpr int KSB = (16 * RV > 32 * TST ? 16 * RV : 32 * TST);  // bf16 per wave staging block
  constexpr int SEJ = 48;                 // scale_embed rows staged (J <= 48)
  constexpr int NTSE = 3 * DB;            // 16x16 tiles of dse^T [D x 48]
  constexpr int TPW = (NTSE + 3) / 4;     // ... per wave
  constexpr bool QROWS = HAS_SE || DG;    // the query rows are needed whole-row (dse, long-range q.k)
  constexpr float kLog2e = 1.4426950408889634f;

  __shared__ __align__(16) bf16_t sK[WIN * RV];        // dense-window K rows
  __shared__ __align__(16) bf16_t sV[WIN * RV];        // dense-window V rows
  // Wave-private staging block: with scale_embed first the dense-tap table
  // T[i][j] = log2e (bias_j + c q_i.se_j); then the two rounds that turn dq into row layout;
  // then, with scale_embed, the wave's Q rows (read by every wave for dse).
  __shared__ __align__(16) bf16_t sKs[4][HAS_SE ? KSB : 16 * RV];
  // scale_embed rows as two bf16 planes, hi = bf16(se) and lo = bf16(se - hi): q.se and
  // SE^T dS then carry se to about 2^-17 relative, as the fp32 se of the reference.
  __shared__ __align__(16) bf16_t sSE[HAS_SE ? SEJ * RV : 8];
  __shared__ __align__(16) bf16_t sSElo[HAS_SE ? SEJ * RV : 8];
  // [query][tap] per wave: u of the long-range taps (pass 1), then dS.  It lives in the V window
  // once the band is done (D >= 64), which keeps the workgroup's LDS small enough for four
  // workgroups per CU (three with scale_embed).
  constexpr bool TBL_IN_V = WIN * RV * 2 >= 4 * 16 * TS * 4;
  __shared__ __align__(16) float sDSst[TBL_IN_V ? 4 : 4 * 16 * TS];
  // c q.k per (query, tap), for dg only: dynamic LDS, present when score_gain's gradient is
  // requested.
  extern __shared__ __align__(16) float sDyn[];
  float* const sRAW = sDyn;
  __shared__ float sBias2[kMaxTaps];
  __shared__ float sGain[kMaxTaps];
  __shared__ float sDp[4][16];            // per wave: D' of its rows (the da sum)

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
               : "s"(p.q), "s"(p.k), "s"(p.v), "s"(p.dout), "s"(p.lse), "s"(p.pos_bias), "s"(p.if_gain),
                 "s"(p.alpha_lr));
  const int lb = xcd_logical_block(blockIdx.x, nblk);
  // Workgroup lb: tile lb % n_chunks of head h of batch group grp ((grp * H + h) * n_chunks + tile).
  const int gh = lb / p.n_chunks, tile = lb - gh * p.n_chunks;
  const int grp = gh / p.H, h = gh - grp * p.H;
  const int N = p.N, J = p.taps.J, W = p.taps.W;
  const int NS = NSC > 0 ? NSC : J - W - 1;
  const float c = p.scale, c2 = p.scale * kLog2e;
  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const bool se_grad = p.part_se != nullptr;
  constexpr bool g_grad = DG;
  const int qsn = (int)p.qs.n, ksn = (int)p.ks.n, vsn = (int)p.vs.n, dosn = (int)p.dos.n;



  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int dl_s[NSM];
  load_sparse_deltas(p.taps, dl_s);

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
  // in the V window gets them after the band.  Thread t clears row t % 64 from column J + t / 64
  // on, every fourth column.
  for (int j = J + (tid >> 6); j < 48; j += kBlock / 64) {
    if (!TBL_IN_V) sDS[(tid & 63) * TS + j] = 0.f;
    if (g_grad) sRAW[(tid & 63) * TS + j] = 0.f;
  }
  float* sDSw = sDS + w * 16 * TS;
  float* sRAWw = sRAW + w * 16 * TS;  // dereferenced only when g_grad
  bf16_t* sKsw = sKs[w];
  float* sTw = reinterpret_cast<float*>(sKsw);

  // The parameter-gradient partials of the workgroup's (b,h) slices, summed in batch order.  With
  // scale_embed a workgroup takes its head and tile in p.batches_per_block batches, so that its
  // [J x D] dse partial covers that many times 64 queries (the partials are as large as a tile's
  // dS otherwise); without it one batch.
  float acc_bias = 0.f, acc_gain = 0.f, acc_if = 0.f;
  f32x4_t accSE[HAS_SE ? TPW : 1];  // this wave's dse^T tiles w, w+4, ...
#pragma unroll
  for (int k = 0; k < (HAS_SE ? TPW : 1); ++k) accSE[k] = zero4();
  const int bpb = HAS_SE ? p.batches_per_block : 1;
  for (int tk = 0; tk < bpb; ++tk) {
  const int b = grp * bpb + tk;
  if (HAS_SE && b >= p.B) break;  // one batch per workgroup otherwise: the grid is exact
  const int bh = b * p.H + h;
  const __amdgpu_buffer_rsrc_t rQ = slice_rsrc(static_cast<const bf16_t*>(p.q) + b * p.qs.b + h * p.qs.h, p.qs.n, N, D);
  const __amdgpu_buffer_rsrc_t rK = slice_rsrc(static_cast<const bf16_t*>(p.k) + b * p.ks.b + h * p.ks.h, p.ks.n, N, D);
  const __amdgpu_buffer_rsrc_t rV = slice_rsrc(static_cast<const bf16_t*>(p.v) + b * p.vs.b + h * p.vs.h, p.vs.n, N, D);
  const __amdgpu_buffer_rsrc_t rO = slice_rsrc(static_cast<const bf16_t*>(p.dout) + b * p.dos.b + h * p.dos.h, p.dos.n, N, D);
  bf16_t* dqb = static_cast<bf16_t*>(p.dq) + b * p.dqs.b + h * p.dqs.h;
  const long long rowbase = ((long long)b * p.H + h) * N;
  // Lane indices and everything derived from them are formed anew for each tile (from an opaque
  // copy of the thread index): hoisted out of the tile loop, the per-lane addresses stayed live
  // across it and spilled.
  const int l = opaque(tid) & 63, i = l & 15, g = l >> 4;
  // The diagonal lane of query i (group i/4, register i%4) owns its long-range taps: it reads
  // their forward weights, forms their dS and files them in the wave's table, which the row
  // layout's lanes read for pass 2.
  const bool diag = g == (i >> 2);
  const int qlane = opaque(i * qsn + 8 * g), olane = opaque(i * dosn + 8 * g);
  // Row-chunk layout for the long-range rows and their dot partners.
  int qlaneR[CHW], olaneR[CHW], klaneR[CHW], vlaneR[CHW];
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    qlaneR[u] = opaque(rc_lane<D>(l, u, qsn));
    olaneR[u] = opaque(rc_lane<D>(l, u, dosn));
    klaneR[u] = opaque(rc_lane<D>(l, u, ksn));
    vlaneR[u] = opaque(rc_lane<D>(l, u, vsn));
  }
  const int n0 = tile * QT;
  const int n0w = n0 + 16 * w;
  const int n = n0w + i;  // query row of this lane's MFMA column
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
  uint4 oR[CHW];
  [[maybe_unused]] uint4 qR[QROWS ? CHW : 1];
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    oR[u] = bload16(rO, n0w * dosn + olaneR[u]);
    if constexpr (QROWS) qR[u] = bload16(rQ, n0w * qsn + qlaneR[u]);
  }
  // Unconditional (a row past N reads row N - 1 and is masked below): a load under the row
  // test was waited for inside the branch, before the long-range loads could be issued.
  const float lse_ld = p.lse[rowbase + (row_ok ? n : N - 1)];
  // The forward's long-range weights of this lane's query ([b,h][tap][query] fp32), on the
  // diagonal lane of a row below N; every other lane's offset lies past the buffer resource (one
  // over the (b,h)'s NS x N weights, NS N 4 < 2^31 bytes), which returns zeros.  The tap's
  // offset t N 4 rides in the scalar offset: lanes in range stay in range with it, lanes out of
  // range stay out.
  float als[NSM];
  {
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.alpha_lr + (long long)bh * NS * N), (short)0, NS * N * 4, 0x00020000);
    const unsigned off = diag && row_ok ? (unsigned)n * 4u : 0x80000000u;
#pragma unroll
    for (int t = 0; t < NSM; ++t) {
      als[t] = 0.f;
      if (NSC > 0 || t < NS)
        als[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rA, off, t * N * 4, 0));
    }
  }
  // Long-range rows, one ring of PF slots for both passes: block k of the sequence
  // V(0..NSM-1), K(0..NSM-1) goes to slot k % PF, so pass 1 takes tap t's V rows from slot
  // t % PF and pass 2 its K rows from slot (NSM + t) % PF.  Every index is a compile-time
  // constant (the generic-table form, whose tap count NS is known only at run time, skips the
  // blocks of taps t >= NS instead of shifting the K blocks down): indexed by NS, the ring and
  // the offsets went to scratch memory.  Rows n0w - delta + 0..15, in the row-chunk layout.
  uint4 rS[PF][CHW];
  auto load_rows = [&](int k) {
    const bool isv = k < NSM;
    const int t = isv ? k : k - NSM;
    if (NSC == 0 && t >= NS) return;
    const int m0 = n0w - dl_s[t];
#pragma unroll
    for (int u = 0; u < CHW; ++u)
      rS[k % PF][u] = isv ? bload16(rV, m0 * vsn + vlaneR[u]) : bload16(rK, m0 * ksn + klaneR[u]);
  };
#pragma unroll
  for (int k = 0; k < PF; ++k)
    if (k < 2 * NSM) load_rows(k);

  if (!HAS_SE && tid < J) {
    sBias2[tid] = bias_ld * kLog2e;
    sGain[tid] = gain_ld;
  }
  if (tk > 0) __syncthreads();  // the previous slice's reads of the windows and tables are done
#pragma unroll
  for (int u = 0; u < CWIN; ++u) {
    const int ci = tid + u * kBlock;
    if (ci < WIN * CPS) {
      st16(sK + (ci / CPS) * RV + (ci % CPS) * 8, wk[u]);
      st16(sV + (ci / CPS) * RV + (ci % CPS) * 8, wv[u]);
    }
  }
  __syncthreads();

  // ---- 1. Dense band: S^T = K Q^T, U^T = V dOut^T. ----
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
      if (16 * jb > W) continue;
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

  // Dense weights and u; D' collects alpha u of every tap of this lane's query column.
  float al[12], uu[12];
  float dlane = 0.f;
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
      // c q.k for dg goes to the table now (frees the score registers).
      if (g_grad && (unsigned)dl <= (unsigned)W) sRAWw[i * TS + dl] = c * accS[kk][r];
    }
  }
  if constexpr (TBL_IN_V) {
    __syncthreads();  // every wave's band reads of sV are done: the tables move in
    for (int j = J + g; j < 48; j += 4) sDSw[i * TS + j] = 0.f;
  }

  // ---- 2. Long-range pass 1: u_j = dOut . v_j of each row, into the table (no wait per tap). ----
#pragma unroll
  for (int t = 0; t < NSM; ++t) {
    if (NSC > 0 || t < NS) {
#pragma unroll
      for (int rg = 0; rg < CHW / CPL; ++rg) {
        float uv = dot8_bf16(oR[rg * CPL], rS[t % PF][rg * CPL], 0.f);
#pragma unroll
        for (int pc = 1; pc < CPL; ++pc) uv += dot8_bf16(oR[rg * CPL + pc], rS[t % PF][rg * CPL + pc], 0.f);
        uv = group_sum<CPRP>(uv);
        if (l % CPRP == 0) sDSw[rc_row<D>(l, rg * CPL) * TS + W + 1 + t] = uv;
      }
    }
    // (In the generic-table form the iterations t >= NS consume nothing and issue the first
    // K blocks of pass 2.)
    if (t + PF < 2 * NSM) load_rows(t + PF);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): every row's u is in the table
  __builtin_amdgcn_wave_barrier();
  float uus[NSM];
#pragma unroll
  for (int t = 0; t < NSM; ++t) {
    uus[t] = 0.f;
    if (NSC > 0 || t < NS) {
      uus[t] = sDSw[i * TS + W + 1 + t];
      dlane = fmaf(als[t], uus[t], dlane);  // als[t] is zero off the diagonal
    }
  }
  const float Dp = col_sum(dlane);  // D' = dOut . o (pre-gain o) for query n

  // ---- 3. dq = X + SE^T (c dS)^T, X = sum_j (c g_j dS_j) k_j. ----
  f32x4_t X[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) X[db] = zero4();
  const float ca = c * a;
#pragma unroll
  for (int kk = 0; kk < 3; ++kk) {
    float wq[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dl = dl0 - 16 * kk - r;
      const bool in = (unsigned)dl <= (unsigned)W;
      const int j = in ? dl : 0;
      const float du = al[4 * kk + r] * (uu[4 * kk + r] - Dp);
      if (in) sDSw[i * TS + dl] = a * du;  // every entry j <= W is written (zero where masked)
      wq[r] = sGain[j] * ca * du;
    }
    // The weights as bf16 hi + lo pairs: the products keep the weights' fp32 precision.
    s16x4_t bw, bwl;
    split_bf16x4(wq[0], wq[1], wq[2], wq[3], bw, bwl);
    const bf16_t* kr = sK + (16 * w + 16 * kk + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const s16x4_t at = lds_read_tr16(kr + 16 * db);
      X[db] = mfma_16x16x16(at, bw, X[db]);
      X[db] = mfma_16x16x16(at, bwl, X[db]);
    }
  }

  // dS of every long-range pair, on the query's diagonal lane: into the table (for the SE term,
  // the parameter sums and pass 2) and, with a alpha_j, to launch 2's weights.
  {
    // One buffer resource over the (b,h)'s NS x N weight dwords: a lane off the diagonal or past
    // N stores past its end, which the range check drops.
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<unsigned*>(p.lrw) + (long long)bh * NS * N, (short)0, NS * N * 4, 0x00020000);
    const unsigned woff = diag && row_ok ? (unsigned)n * 4u : 0x80000000u;
#pragma unroll
    for (int t = 0; t < NSM; ++t) {
      if (NSC > 0 || t < NS) {
        const int j = W + 1 + t;
        const float ds = a * als[t] * (uus[t] - Dp);  // zero for masked taps and rows past N
        if (diag) sDSw[i * TS + j] = ds;
        __builtin_amdgcn_raw_buffer_store_b32(cvt_pk_bf16(c * sGain[j] * ds, a * als[t]), rW, woff,
                                              t * N * 4, 0);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's table is complete
  __builtin_amdgcn_wave_barrier();

  if constexpr (HAS_SE) {
    // SE^T (c dS)^T from this wave's own table rows: dq's scale_embed term.
#pragma unroll
    for (int jb = 0; jb < 3; ++jb) {
      const float4 d4 = *reinterpret_cast<const float4*>(sDSw + i * TS + 16 * jb + 4 * g);
      s16x4_t bs, bsl;
      split_bf16x4(c * d4.x, c * d4.y, c * d4.z, c * d4.w, bs, bsl);
      const int so = (16 * jb + 4 * g + (i >> 2)) * RV + 4 * (i & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const s16x4_t sh = lds_read_tr16(sSE + so + 16 * db);
        X[db] = mfma_16x16x16(sh, bs, X[db]);
        X[db] = mfma_16x16x16(sh, bsl, X[db]);
        X[db] = mfma_16x16x16(lds_read_tr16(sSElo + so + 16 * db), bs, X[db]);
      }
    }
  }

  // X (MFMA layout: lane (i, g) holds query i, d = 16 db + 4 g + 0..3) -> row layout (lane: row
  // rc_row, d = 8 rc_chunk + 0..7), fp32, in two rounds of DP/2 columns through the wave's staging
  // block (row stride DP/2 + 4 floats: conflict-free 16-byte writes and reads; a round fills the
  // block exactly).
  float xacc[CHW][8];
  {
    constexpr int HC = G_::DP / 2;  // columns per round
    constexpr int CS = HC + 4;
    constexpr int CPH = HC / 8;     // row chunks per round
    static_assert(16 * CS * 4 <= (HAS_SE ? KSB : 16 * RV) * 2, "a round fits the staging block");
    float* const cvt = reinterpret_cast<float*>(sKsw);
#pragma unroll
    for (int u = 0; u < CHW; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) xacc[u][e] = 0.f;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int db = hf * HC / 16; db < (hf + 1) * HC / 16 && db < DB; ++db)
        *reinterpret_cast<float4*>(cvt + i * CS + 16 * db - hf * HC + 4 * g) =
            make_float4(X[db][0], X[db][1], X[db][2], X[db][3]);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the quads are written
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int u = 0; u < CHW; ++u) {
        const int cc = rc_chunk<D>(l, u);
        if (cc < CPR && cc / CPH == hf) {
          const float* src = cvt + rc_row<D>(l, u) * CS + 8 * (cc - hf * CPH);
          const float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
          xacc[u][0] = lo.x; xacc[u][1] = lo.y; xacc[u][2] = lo.z; xacc[u][3] = lo.w;
          xacc[u][4] = hi.x; xacc[u][5] = hi.y; xacc[u][6] = hi.z; xacc[u][7] = hi.w;
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the rows are read before the next round
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---- Long-range pass 2, K rows: dq_n += c g_j dS_j(n) k_j, one scaled key row per query row. ----
  // No contraction: fp32 FMAs in the row layout the gathered rows arrive in, against the exact
  // fp32 weight (read from the table by each row's lanes, one tap ahead), with no LDS staging and
  // no wait per tap.
  {
    float wnx[CHW];
    auto read_w = [&](int t) {
      const float cg = c * sGain[W + 1 + t];
#pragma unroll
      for (int u = 0; u < CHW; ++u) wnx[u] = cg * sDSw[rc_row<D>(l, u) * TS + W + 1 + t];
    };
    read_w(0);
#pragma unroll
    for (int t = 0; t < NSM; ++t) {
      if (NSC > 0 || t < NS) {
        const int slot = (NSM + t) % PF;
        float wc[CHW];
#pragma unroll
        for (int u = 0; u < CHW; ++u) wc[u] = wnx[u];
        if (t + 1 < NS) read_w(t + 1);
#pragma unroll
        for (int u = 0; u < CHW; ++u) {
          const uint4 kv = rS[slot][u];
          const unsigned kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            xacc[u][2 * e] = fmaf(wc[u], __builtin_bit_cast(float, kw[e] << 16), xacc[u][2 * e]);
            xacc[u][2 * e + 1] = fmaf(wc[u], __builtin_bit_cast(float, kw[e] & 0xffff0000u), xacc[u][2 * e + 1]);
          }
        }
        if constexpr (DG) {
#pragma unroll
          for (int rg = 0; rg < CHW / CPL; ++rg) {
            float qk = dot8_bf16(qR[rg * CPL], rS[slot][rg * CPL], 0.f);
#pragma unroll
            for (int pc = 1; pc < CPL; ++pc) qk += dot8_bf16(qR[rg * CPL + pc], rS[slot][rg * CPL + pc], 0.f);
            qk = group_sum<CPRP>(qk);
            if (l % CPRP == 0) sRAWw[rc_row<D>(l, rg * CPL) * TS + W + 1 + t] = c * qk;
          }
        }
        // The tap's sums are due here (the empty asm pins them: pure arithmetic is otherwise sunk
        // past every later tap's loads), and each tap's loads stay in its own iteration.
#pragma unroll
        for (int u = 0; u < CHW; ++u)
#pragma unroll
          for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(xacc[u][e]));
        __builtin_amdgcn_sched_barrier(0);
        if (t + PF < NSM) load_rows(NSM + t + PF);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  if constexpr (HAS_SE) {
    // The wave's Q rows (natural order) replace the conversion rounds in its staging block, for
    // dse once every table is done.
    if (se_grad) {
#pragma unroll
      for (int u = 0; u < CHW; ++u)
        if (rc_valid<D>(l, u)) st16(sKsw + rc_row<D>(l, u) * RV + rc_chunk<D>(l, u) * 8, qR[u]);
    }
  }
  if (g == 0) sDp[w][i] = row_ok ? Dp : 0.f;
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();

  // dbias / dg column sums of this wave's 16 table rows (its own writes, complete above),
  // and the wave's sum of D' (for da).
  if (l < J) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float ds = sDSw[r * TS + l];
      acc_bias += ds;
      if (g_grad) acc_gain = fmaf(ds, sRAWw[r * TS + l], acc_gain);
    }
  }
  if (l == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_if += sDp[w][r];
  }

  if constexpr (HAS_SE) {
    __syncthreads();  // all waves' tables and Q rows are complete
    // dse partial on the MFMA: dSE^T (d x j) += Q^T (d x q) dS (q x j) over the tile's 64
    // queries; wave w owns the output tiles w, w+4, ... of the 3 x DB grid.
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

  // dq leaves as whole rows straight from the row layout: 16-byte pieces per lane.
#pragma unroll
  for (int u = 0; u < CHW; ++u) {
    const int rr = rc_row<D>(l, u), cc = rc_chunk<D>(l, u);
    if (n0w + rr < N && cc < CPR) {
      uint4 o;
      o.x = cvt_pk_bf16(xacc[u][0], xacc[u][1]); o.y = cvt_pk_bf16(xacc[u][2], xacc[u][3]);
      o.z = cvt_pk_bf16(xacc[u][4], xacc[u][5]); o.w = cvt_pk_bf16(xacc[u][6], xacc[u][7]);
      st16(dqb + (n0w + rr) * p.dqs.n + 8 * cc, o);
    }
  }
  if (row_ok && g == 0) p.dpre[rowbase + n] = Dp;
  }  // tiles
  const int l = tid & 63, i = l & 15, g = l >> 4;

  // The four waves' partial sums meet in their own (now free) table blocks; one partial row per
  // workgroup, summed in wave order.
  {
    __syncthreads();  // every wave's reads of the tables (column sums, dse, SE term) are done
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
  if (p.part_gain) {  // the score gain's gradient, with its dg table in dynamic LDS
    const size_t dyn = sizeof(float) * 4 * 16 * kDqTableStride;
    switch (p.taps.J - p.taps.W - 1) {
      case 11: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 11, true>), dim3(nb), dim3(kBlock), dyn, st, p); break;
      case 13: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 13, true>), dim3(nb), dim3(kBlock), dyn, st, p); break;
      case 14: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 14, true>), dim3(nb), dim3(kBlock), dyn, st, p); break;
      default: hipLaunchKernelGGL((bwd_dq_mfma_kernel<D, HAS_SE, 0, true>), dim3(nb), dim3(kBlock), dyn, st, p); break;
    }
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
  // Several tiles per workgroup only with scale_embed (its dse partials).
  if (p.tiles_per_block != 1 || p.batches_per_block < 1 ||
      (p.batches_per_block != 1 && !(p.scale_embed || p.part_se)))
    return hipErrorInvalidValue;
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
