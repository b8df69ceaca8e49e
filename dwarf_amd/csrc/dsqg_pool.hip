// Causal-mean pool with a sigmoid gate over [B,N,C] tensors: the interference branch of a
// DWARF block (train/train_2048_condU.py:289-292):
//
//     pool[b,n,c]  = (sum_{m<=n} x[b,m,c]) / (n + 1)
//     out[b,n,c]   = sigmoid(gate_pre[b,n,c]) * pool[b,n,c]
//
// and its backward (dout = d out):
//
//     dgate_pre    = dout * pool * s * (1 - s),             s = sigmoid(gate_pre)
//     dx[b,m,c]    = sum_{n>=m} dout[b,n,c] * s[b,n,c] / (n + 1)
//
// Both are column scans along N, HBM-bound: every element is read and written once in the
// scan pass.  The scan is split in two launches over row chunks of L rows:
//   1. chunk sums: per (b, chunk, channel) the sum of x over the chunk (and, backward, of
//      dout * s / (n+1)), fp32, into the workspace;
//   2. scan: each workgroup adds the sums of the chunks before it (after it, for the
//      backward's suffix sum), scans its own rows and writes the outputs.
// A workgroup is 16 channel groups (4 channels per lane: one 128-byte bf16 row segment per
// 16 lanes) times 16 row lanes; a row lane holds RPL consecutive rows in registers, so a chunk
// is L = 16 * RPL rows.  Across the row lanes of a wave the sums and scans are lane shuffles
// (strides 16 and 32 lanes), across the four waves one LDS exchange; a lane reads every 16th
// earlier chunk sum.  Every sum runs in a fixed order: results are deterministic.
//
// Element types are per tensor (f32, bf16, f16) and uniform per launch.  A launch whose tensors
// are all bf16 runs kernels compiled for that type; any other mix switches at each load on the
// tensor's type (a scalar branch), which splits the loads into separately waited groups and
// costs registers (at [8, 2048, 768] bf16: forward 24.5 -> 18.6 us, backward 58.1 -> 40.1 us
// for the compiled-type kernels).  As torch computes sigmoid in the gate's dtype, s is rounded
// to that dtype before it is used; all arithmetic is fp32, with 1/(n+1) and the sigmoid's
// reciprocal from v_rcp_f32 (1 ulp).
#include "../../include/dsqg.h"
#include "dsqg_common.hpp"

namespace dsqg {
namespace {

constexpr int kCpl = 4;                     // channels per lane
constexpr int kPoolCgt = 16;                // channel groups (lanes across channels) per workgroup
constexpr int kPoolCh = kPoolCgt * kCpl;    // 64 channels per workgroup
constexpr int kPoolRl = kBlock / kPoolCgt;  // 16 row lanes per workgroup, 4 per wave
constexpr int kWaveRl = 64 / kPoolCgt;

struct PoolParams {
  const void* x;  long long xs_b, xs_n;
  const void* g;  long long gs_b, gs_n;
  const void* dy; long long ys_b, ys_n;   // dout (backward only)
  void* out;      long long os_b, os_n;   // forward output
  void* dx;       long long dxs_b, dxs_n; // backward outputs (either may be null)
  void* dg;       long long dgs_b, dgs_n;
  float* px;      // [B][nchunks][C] chunk sums of x
  float* pp;      // [B][nchunks][C] chunk sums of dout * s / (n+1) (backward)
  int B, N, C;
  int nchunks, ctiles, L;
  int xdt, gdt, ydt, odt;  // element types (DSQG_F32 / DSQG_BF16 / DSQG_F16)
};

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}
__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)a) |
         ((uint32_t)__builtin_bit_cast(unsigned short, (_Float16)b) << 16);
}
// Two floats -> packed bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t r;
  r[0] = (__bf16)a;
  r[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

// x rounded to element type dt.
__device__ __forceinline__ float round_to(int dt, float x) {
  if (dt == DSQG_BF16) return (float)(__bf16)x;
  if (dt == DSQG_F16) return (float)(_Float16)x;
  return x;
}

__device__ __forceinline__ float sigmoid_as(int dt, float g) {
  return round_to(dt, __builtin_amdgcn_rcpf(1.0f + __expf(-g)));
}

// Element type of a launch's tensors: DT when the launch fixes one type for all of them (the
// type branches then fold away at compile time), else the tensor's own runtime type (DT = -1).
template <int DT>
__device__ __forceinline__ int dt_of(int runtime_dt) { return DT >= 0 ? DT : runtime_dt; }

// The kernel arguments a prologue needs, requested in one round trip: they pass through one
// empty asm statement that everything after it depends on (otherwise the compiler waits for
// the grid constants, divides, and only then asks for the pointers, strides and sizes: three
// dependent scalar round trips before the first row load).
__device__ __forceinline__ void pool_args_at_once(PoolParams& p) {
  asm volatile("" : "+s"(p.ctiles), "+s"(p.nchunks), "+s"(p.N), "+s"(p.C), "+s"(p.L)
               : "s"(p.x), "s"(p.g), "s"(p.dy), "s"(p.px), "s"(p.pp), "s"(p.xs_b), "s"(p.xs_n),
                 "s"(p.gs_b), "s"(p.gs_n), "s"(p.ys_b), "s"(p.ys_n));
}

// Lane coordinates: tid = rl * 16 + cgl, so a wave holds 16 channel groups x 4 row lanes.
struct PoolLane {
  int b, chunk, cgl, rl, c;  // c: first channel of this lane; active iff c < C
  bool active;
  int row0;                  // first of this lane's RPL rows
};

template <int RPL>
__device__ __forceinline__ PoolLane pool_lane(const PoolParams& p) {
  PoolLane q;
  const int bid = blockIdx.x;
  const int ct = bid % p.ctiles;
  const int bc = bid / p.ctiles;
  q.chunk = bc % p.nchunks;
  q.b = bc / p.nchunks;
  const int tid = threadIdx.x;
  q.cgl = tid & (kPoolCgt - 1);
  q.rl = tid / kPoolCgt;
  q.c = (ct * kPoolCgt + q.cgl) * kCpl;
  q.active = q.c < p.C;
  q.row0 = q.chunk * p.L + q.rl * RPL;
  return q;
}

// Rows of one [B,N,C] operand for this lane: a buffer resource over the batch's slice (its exact
// extent, so rows >= N read as zero and stores there are dropped), the byte offset of the lane's
// first row and channel, and the row stride in bytes (uniform, passed as the scalar offset).
struct TensorRows {
  __amdgpu_buffer_rsrc_t r;
  unsigned lane, rstep;
  int dt;
};

__device__ __forceinline__ TensorRows rows_of(const void* base, long long sb, long long sn, int dt,
                                              const PoolParams& p, const PoolLane& q) {
  const long long es = dt == DSQG_F32 ? 4 : 2;
  TensorRows t;
  const char* slice = static_cast<const char*>(base) + (long long)q.b * sb * es;
  const int ext = p.N > 0 ? (int)(((long long)(p.N - 1) * sn + p.C) * es) : 0;
  t.r = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(slice), (short)0, ext, 0x00020000);
  t.lane = (unsigned)(((long long)q.row0 * sn + q.c) * es);
  t.rstep = (unsigned)(sn * es);
  t.dt = dt;
  return t;
}

// Channels c..c+3 of row row0 + r (zero beyond the slice).
__device__ __forceinline__ void tload(const TensorRows& t, int r, float (&v)[kCpl]) {
  if (t.dt == DSQG_F32) {
    const float4 a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(t.r, t.lane, r * t.rstep, 0));
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    return;
  }
  const uint2 w = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(t.r, t.lane, r * t.rstep, 0));
  if (t.dt == DSQG_BF16) {
    v[0] = __uint_as_float(w.x << 16); v[1] = __uint_as_float(w.x & 0xffff0000u);
    v[2] = __uint_as_float(w.y << 16); v[3] = __uint_as_float(w.y & 0xffff0000u);
  } else {
    v[0] = f16_to_f32(w.x & 0xffffu); v[1] = f16_to_f32(w.x >> 16);
    v[2] = f16_to_f32(w.y & 0xffffu); v[3] = f16_to_f32(w.y >> 16);
  }
}

// A lane's RPL rows x kCpl channels kept for a later pass over the rows.  PACK (the tensor is
// bf16, and so is every value kept): as packed bf16 pairs, half the registers, one VALU
// instruction to unpack an element.  Otherwise as floats.
template <int RPL, bool PACK>
struct RowBuf {
  float v[RPL][kCpl];
  // Loads row r into the buffer and returns it in a.
  __device__ __forceinline__ void load(const TensorRows& t, int r, float (&a)[kCpl]) {
    tload(t, r, v[r]);
#pragma unroll
    for (int e = 0; e < kCpl; ++e) a[e] = v[r][e];
  }
  __device__ __forceinline__ void set(int r, const float (&a)[kCpl]) {
#pragma unroll
    for (int e = 0; e < kCpl; ++e) v[r][e] = a[e];
  }
  __device__ __forceinline__ float get(int r, int e) const { return v[r][e]; }
};

template <int RPL>
struct RowBuf<RPL, true> {
  uint32_t w[RPL][2];
  __device__ __forceinline__ void load(const TensorRows& t, int r, float (&a)[kCpl]) {
    const uint2 u = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(t.r, t.lane, r * t.rstep, 0));
    w[r][0] = u.x; w[r][1] = u.y;
#pragma unroll
    for (int e = 0; e < kCpl; ++e) a[e] = get(r, e);
  }
  __device__ __forceinline__ void set(int r, const float (&a)[kCpl]) {  // a: bf16 values
    w[r][0] = pack2_bf16(a[0], a[1]);
    w[r][1] = pack2_bf16(a[2], a[3]);
  }
  __device__ __forceinline__ float get(int r, int e) const {
    const uint32_t u = w[r][e >> 1];
    return __uint_as_float((e & 1) ? (u & 0xffff0000u) : (u << 16));
  }
};

// Store channels c..c+3 of row row0 + r (dropped beyond the slice).  Callers skip inactive
// lanes, whose channels lie past C (inside another row's stride gap).  Stores are at most 8
// bytes: after a wider VMEM store the hardware needs one wait state before a VALU instruction
// overwrites the store's data registers, and the compiler was seen to omit it where the store
// ends a basic block (the next block's first add rewrote the data, so the stored value already
// held the following row's term).
__device__ __forceinline__ void tstore(const TensorRows& t, int r, const float (&v)[kCpl]) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  if (t.dt == DSQG_F32) {
    const u32x2 lo = {__float_as_uint(v[0]), __float_as_uint(v[1])};
    const u32x2 hi = {__float_as_uint(v[2]), __float_as_uint(v[3])};
    __builtin_amdgcn_raw_buffer_store_b64(lo, t.r, t.lane, r * t.rstep, 0);
    __builtin_amdgcn_raw_buffer_store_b64(hi, t.r, t.lane + 8, r * t.rstep, 0);
    return;
  }
  u32x2 w;
  if (t.dt == DSQG_BF16) {
    w[0] = pack2_bf16(v[0], v[1]);
    w[1] = pack2_bf16(v[2], v[3]);
  } else {
    w[0] = pack2_f16(v[0], v[1]);
    w[1] = pack2_f16(v[2], v[3]);
  }
  __builtin_amdgcn_raw_buffer_store_b64(w, t.r, t.lane, r * t.rstep, 0);
}

// Total over the 16 row lanes of each of this lane's channels, returned to every lane:
// shuffles over the wave's 4 row lanes (lane strides 16, 32), then the four wave totals
// through sW (4 x 64 floats).  Starts with a barrier, so sW may be reused back to back.
__device__ __forceinline__ void rl_total(float (&v)[kCpl], float* sW) {
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, cgl = tid & (kPoolCgt - 1);
#pragma unroll
  for (int off = kPoolCgt; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < kCpl; ++e) v[e] += __shfl_xor(v[e], off, 64);
  __syncthreads();
  if (l < kPoolCgt) {
#pragma unroll
    for (int e = 0; e < kCpl; ++e) sW[w * kPoolCh + cgl * kCpl + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kCpl; ++e)
    v[e] = (sW[cgl * kCpl + e] + sW[kPoolCh + cgl * kCpl + e]) +
           (sW[2 * kPoolCh + cgl * kCpl + e] + sW[3 * kPoolCh + cgl * kCpl + e]);
}

// Exclusive scan over the 16 row lanes of each channel: the sum of v over the row lanes before
// this one (SUFFIX: after it).  Shuffle scan within the wave, wave totals through sW.
template <bool SUFFIX>
__device__ __forceinline__ void rl_exclusive_scan(float (&v)[kCpl], float* sW) {
  const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, cgl = tid & (kPoolCgt - 1);
  const int lr = l / kPoolCgt;  // row lane within the wave
  float inc[kCpl];
#pragma unroll
  for (int e = 0; e < kCpl; ++e) inc[e] = v[e];
#pragma unroll
  for (int off = kPoolCgt; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < kCpl; ++e) {
      const float t = SUFFIX ? __shfl_down(inc[e], off, 64) : __shfl_up(inc[e], off, 64);
      if (SUFFIX ? (l + off < 64) : (l >= off)) inc[e] += t;
    }
  }
  __syncthreads();
  if (lr == (SUFFIX ? 0 : kWaveRl - 1)) {
#pragma unroll
    for (int e = 0; e < kCpl; ++e) sW[w * kPoolCh + cgl * kCpl + e] = inc[e];
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kCpl; ++e) {
    float base = 0.f;
    for (int k = 0; k < 4; ++k)
      if (SUFFIX ? (k > w) : (k < w)) base += sW[k * kPoolCh + cgl * kCpl + e];
    v[e] = base + (inc[e] - v[e]);
  }
}

// Sum over chunks k = first, first + 16, ... < last of a [B][nchunks][C] partial array, in
// two steps: begin() issues the first two loads (chunks first, first + 16) so
// that they travel with the row loads that follow, finish() adds them and any further chunks.
struct ChunkCarry {
  float4 a0, a1;
  int next, end;
  __device__ __forceinline__ void begin(const float* part, const PoolParams& p, const PoolLane& q,
                                        int first, int last) {
    end = q.active ? last : first;
    const float* base = part + (long long)q.b * p.nchunks * p.C + q.c;
    a0 = first < end ? *reinterpret_cast<const float4*>(base + (long long)first * p.C) : make_float4(0.f, 0.f, 0.f, 0.f);
    a1 = first + kPoolRl < end ? *reinterpret_cast<const float4*>(base + (long long)(first + kPoolRl) * p.C)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    next = first + 2 * kPoolRl;
  }
  __device__ __forceinline__ void finish(const float* part, const PoolParams& p, const PoolLane& q,
                                         float (&acc)[kCpl]) const {
    acc[0] = a0.x + a1.x; acc[1] = a0.y + a1.y; acc[2] = a0.z + a1.z; acc[3] = a0.w + a1.w;
    const float* base = part + (long long)q.b * p.nchunks * p.C + q.c;
    for (int k = next; k < end; k += kPoolRl) {
      const float4 a = *reinterpret_cast<const float4*>(base + (long long)k * p.C);
      acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
    }
  }
};

// ---- Pass 1: chunk sums of x (and, backward, of dout * s / (n+1)). -----------------------
template <int RPL, bool BWD, int DT>
__global__ __launch_bounds__(kBlock) void pool_chunk_sum_kernel(PoolParams p) {
  __shared__ float sW[4 * 64];
  pool_args_at_once(p);
  const PoolLane q = pool_lane<RPL>(p);
  const int gdt = dt_of<DT>(p.gdt);
  const TensorRows tx = rows_of(p.x, p.xs_b, p.xs_n, dt_of<DT>(p.xdt), p, q);
  float ax[kCpl], ap[kCpl];
#pragma unroll
  for (int e = 0; e < kCpl; ++e) ax[e] = ap[e] = 0.f;
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    float v[kCpl];
    tload(tx, r, v);
#pragma unroll
    for (int e = 0; e < kCpl; ++e) ax[e] += v[e];
  }
  if constexpr (BWD) {
    const TensorRows tg = rows_of(p.g, p.gs_b, p.gs_n, gdt, p, q);
    const TensorRows ty = rows_of(p.dy, p.ys_b, p.ys_n, dt_of<DT>(p.ydt), p, q);
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      float gv[kCpl], yv[kCpl];
      tload(tg, r, gv);
      tload(ty, r, yv);   // zero beyond N, so those rows add nothing
      const float inv = __builtin_amdgcn_rcpf((float)(q.row0 + r + 1));
#pragma unroll
      for (int e = 0; e < kCpl; ++e) ap[e] += yv[e] * sigmoid_as(gdt, gv[e]) * inv;
    }
  }
  rl_total(ax, sW);
  if constexpr (BWD) rl_total(ap, sW);
  if (q.rl == 0 && q.active) {
    const long long o = ((long long)q.b * p.nchunks + q.chunk) * p.C + q.c;
    *reinterpret_cast<float4*>(p.px + o) = make_float4(ax[0], ax[1], ax[2], ax[3]);
    if constexpr (BWD) *reinterpret_cast<float4*>(p.pp + o) = make_float4(ap[0], ap[1], ap[2], ap[3]);
  }
}

// ---- Pass 2, forward: out = s * (carry + running sum) / (n+1). ----------------------------
template <int RPL, int DT>
__global__ __launch_bounds__(kBlock) void pool_fwd_scan_kernel(PoolParams p) {
  __shared__ float sW[4 * 64];
  pool_args_at_once(p);
  const PoolLane q = pool_lane<RPL>(p);
  const int gdt = dt_of<DT>(p.gdt);
  const TensorRows tx = rows_of(p.x, p.xs_b, p.xs_n, dt_of<DT>(p.xdt), p, q);
  const TensorRows tg = rows_of(p.g, p.gs_b, p.gs_n, gdt, p, q);
  ChunkCarry cc;
  cc.begin(p.px, p, q, q.rl, q.chunk);
  float x[RPL][kCpl], s[RPL][kCpl];
  float run[kCpl];
#pragma unroll
  for (int e = 0; e < kCpl; ++e) run[e] = 0.f;
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    float gv[kCpl];
    tload(tx, r, x[r]);
    tload(tg, r, gv);
#pragma unroll
    for (int e = 0; e < kCpl; ++e) {
      s[r][e] = sigmoid_as(gdt, gv[e]);
      run[e] += x[r][e];
    }
  }
  float carry[kCpl];
  cc.finish(p.px, p, q, carry);
  rl_total(carry, sW);
  rl_exclusive_scan<false>(run, sW);
#pragma unroll
  for (int e = 0; e < kCpl; ++e) run[e] += carry[e];
  const TensorRows to = rows_of(p.out, p.os_b, p.os_n, dt_of<DT>(p.odt), p, q);
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    const float inv = __builtin_amdgcn_rcpf((float)(n + 1));
    float o[kCpl];
#pragma unroll
    for (int e = 0; e < kCpl; ++e) {
      run[e] += x[r][e];
      o[e] = s[r][e] * (run[e] * inv);
    }
    if (q.active) tstore(to, r, o);
  }
}

// ---- Pass 2, backward. ----------------------------------------------------------------------
template <int RPL, int DT>
__global__ __launch_bounds__(kBlock, 4) void pool_bwd_scan_kernel(PoolParams p) {
  __shared__ float sW[4 * 64];
  pool_args_at_once(p);
  const PoolLane q = pool_lane<RPL>(p);
  const int xdt = dt_of<DT>(p.xdt), gdt = dt_of<DT>(p.gdt);
  const TensorRows tx = rows_of(p.x, p.xs_b, p.xs_n, xdt, p, q);
  const TensorRows tg = rows_of(p.g, p.gs_b, p.gs_n, gdt, p, q);
  const TensorRows ty = rows_of(p.dy, p.ys_b, p.ys_n, dt_of<DT>(p.ydt), p, q);
  ChunkCarry ccx, ccp;
  ccx.begin(p.px, p, q, q.rl, q.chunk);
  ccp.begin(p.pp, p, q, q.chunk + 1 + q.rl, p.nchunks);
  constexpr bool kPack = DT == DSQG_BF16;
  RowBuf<RPL, kPack> x, s, y;
  float runx[kCpl], runp[kCpl];
#pragma unroll
  for (int e = 0; e < kCpl; ++e) runx[e] = runp[e] = 0.f;
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    float xv[kCpl], gv[kCpl], yv[kCpl], sv[kCpl];
    x.load(tx, r, xv);
    tload(tg, r, gv);
    y.load(ty, r, yv);   // zero beyond N: those rows add nothing below
#pragma unroll
    for (int e = 0; e < kCpl; ++e) sv[e] = sigmoid_as(gdt, gv[e]);
    s.set(r, sv);
    const float inv = __builtin_amdgcn_rcpf((float)(n + 1));
#pragma unroll
    for (int e = 0; e < kCpl; ++e) {
      runx[e] += xv[e];
      runp[e] += yv[e] * sv[e] * inv;   // dout * s / (n+1), recomputed the same way below
    }
  }
  float cx[kCpl], cp[kCpl];
  ccx.finish(p.px, p, q, cx);
  ccp.finish(p.pp, p, q, cp);
  rl_total(cx, sW);
  rl_total(cp, sW);
  rl_exclusive_scan<false>(runx, sW);
  rl_exclusive_scan<true>(runp, sW);
#pragma unroll
  for (int e = 0; e < kCpl; ++e) {
    runx[e] += cx[e];
    runp[e] += cp[e];
  }
  const TensorRows tdg = rows_of(p.dg ? p.dg : p.x, p.dgs_b, p.dgs_n, gdt, p, q);
  const TensorRows tdx = rows_of(p.dx ? p.dx : p.x, p.dxs_b, p.dxs_n, xdt, p, q);
  // dgate_pre on the way down the rows (prefix sums of x) ...
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    const float inv = __builtin_amdgcn_rcpf((float)(n + 1));
    float o[kCpl];
#pragma unroll
    for (int e = 0; e < kCpl; ++e) {
      const float se = s.get(r, e);
      runx[e] += x.get(r, e);
      o[e] = y.get(r, e) * (runx[e] * inv) * (se * (1.0f - se));
    }
    if (p.dg && q.active) tstore(tdg, r, o);
  }
  // ... and dx on the way up (suffix sums of dout * s / (n+1)).
#pragma unroll
  for (int r = RPL - 1; r >= 0; --r) {
    const int n = q.row0 + r;
    const float inv = __builtin_amdgcn_rcpf((float)(n + 1));
    float o[kCpl];
#pragma unroll
    for (int e = 0; e < kCpl; ++e) {
      runp[e] += y.get(r, e) * s.get(r, e) * inv;
      o[e] = runp[e];
    }
    if (p.dx && q.active) tstore(tdx, r, o);
  }
}

// ---- Host side. ------------------------------------------------------------------------------

struct PoolPlan {
  int rpl, L, nchunks, ctiles;
  long long grid;
};

// 64 channels per workgroup; rows per lane: the most (forward 8, 4, 2, 1; backward from 4) that
// still gives at least 1024 workgroups.  (The backward scan at 4 rows is held to 128 VGPRs, four
// workgroups per CU: the bf16 kernel fits in 119 with its kept rows packed, the runtime-type one
// spills a few; at 2 rows it measured 46.6 against 39.9 us.  The forward at 8 rows: 18.0
// against 19.1 us at [8, 2048, 768] bf16.)
PoolPlan pool_plan(int B, int N, int C, bool bwd) {
  PoolPlan pl;
  pl.ctiles = (C + kPoolCh - 1) / kPoolCh;
  for (int rpl = bwd ? 4 : 8; rpl >= 1; rpl >>= 1) {
    pl.rpl = rpl;
    pl.L = kPoolRl * rpl;
    pl.nchunks = (N + pl.L - 1) / pl.L;
    pl.grid = (long long)B * pl.nchunks * pl.ctiles;
    if (pl.grid >= 1024) break;
  }
  return pl;
}

bool pool_dtype_ok(int dt) { return dt == DSQG_F32 || dt == DSQG_BF16 || dt == DSQG_F16; }
size_t pool_elem(int dt) { return dt == DSQG_F32 ? 4 : 2; }
size_t align256_p(size_t x) { return (x + 255) & ~size_t(255); }

// A [B,N,C] operand: 16-byte aligned base and rows, non-negative batch stride, rows that do
// not overlap (row stride >= C) and a batch slice of less than 2 GiB (the kernels address a
// slice with 32-bit buffer offsets).
int pool_tensor_check(const void* ptr, const int64_t st[2], int dt, int N, int C) {
  if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 15u)) return DSQG_EINVAL;
  const long long es = (long long)pool_elem(dt);
  for (int i = 0; i < 2; ++i)
    if (st[i] < 0 || (st[i] * es) % 16 != 0) return DSQG_EINVAL;
  if (st[1] < C) return DSQG_EINVAL;
  if (((long long)(N - 1) * st[1] + C) * es >= (1ll << 31)) return DSQG_EUNSUPPORTED;
  return DSQG_OK;
}

int pool_shape_ok(int B, int N, int C) {
  if (B < 0 || N < 0 || C <= 0 || C % 8 != 0) return DSQG_EINVAL;
  if ((long long)B * N * C >= (1ll << 40)) return DSQG_EUNSUPPORTED;
  return DSQG_OK;
}

size_t pool_workspace(int B, int N, int C, bool bwd) {
  const PoolPlan pl = pool_plan(B, N, C, bwd);
  const size_t one = align256_p(sizeof(float) * (size_t)B * pl.nchunks * C);
  return bwd ? 2 * one : one;
}

template <int RPL, int DT>
void launch_pool_fwd(const PoolParams& p, unsigned grid, hipStream_t st) {
  hipLaunchKernelGGL((pool_chunk_sum_kernel<RPL, false, DT>), dim3(grid), dim3(kBlock), 0, st, p);
  hipLaunchKernelGGL((pool_fwd_scan_kernel<RPL, DT>), dim3(grid), dim3(kBlock), 0, st, p);
}

template <int RPL, int DT>
void launch_pool_bwd(const PoolParams& p, unsigned grid, hipStream_t st) {
  hipLaunchKernelGGL((pool_chunk_sum_kernel<RPL, true, DT>), dim3(grid), dim3(kBlock), 0, st, p);
  hipLaunchKernelGGL((pool_bwd_scan_kernel<RPL, DT>), dim3(grid), dim3(kBlock), 0, st, p);
}

// All-bf16 launches (the modules' case) run kernels compiled for bf16; any other mix of types
// runs the kernels that switch on each tensor's runtime type.
bool pool_all_bf16(const PoolParams& p) {
  return p.xdt == DSQG_BF16 && p.gdt == DSQG_BF16 && p.ydt == DSQG_BF16 && p.odt == DSQG_BF16;
}

template <int RPL>
void launch_fwd_typed(const PoolParams& p, unsigned grid, hipStream_t st) {
  if (pool_all_bf16(p)) launch_pool_fwd<RPL, DSQG_BF16>(p, grid, st);
  else launch_pool_fwd<RPL, -1>(p, grid, st);
}

template <int RPL>
void launch_bwd_typed(const PoolParams& p, unsigned grid, hipStream_t st) {
  if (pool_all_bf16(p)) launch_pool_bwd<RPL, DSQG_BF16>(p, grid, st);
  else launch_pool_bwd<RPL, -1>(p, grid, st);
}

int run_pool(PoolParams& p, bool bwd, void* ws, size_t ws_bytes, hipStream_t st) {
  const PoolPlan pl = pool_plan(p.B, p.N, p.C, bwd);
  if (pl.grid == 0) return DSQG_OK;
  if (pl.grid > 0x7fffffffll) return DSQG_EUNSUPPORTED;
  const size_t one = align256_p(sizeof(float) * (size_t)p.B * pl.nchunks * p.C);
  if (!ws || (reinterpret_cast<uintptr_t>(ws) & 255u) || ws_bytes < (bwd ? 2 * one : one))
    return DSQG_EWORKSPACE;
  p.px = static_cast<float*>(ws);
  p.pp = bwd ? reinterpret_cast<float*>(static_cast<char*>(ws) + one) : nullptr;
  p.nchunks = pl.nchunks;
  p.ctiles = pl.ctiles;
  p.L = pl.L;
  const unsigned grid = (unsigned)pl.grid;
  if (bwd) {
    if (pl.rpl == 4) launch_bwd_typed<4>(p, grid, st);
    else if (pl.rpl == 2) launch_bwd_typed<2>(p, grid, st);
    else launch_bwd_typed<1>(p, grid, st);
  } else {
    if (pl.rpl == 8) launch_fwd_typed<8>(p, grid, st);
    else if (pl.rpl == 4) launch_fwd_typed<4>(p, grid, st);
    else if (pl.rpl == 2) launch_fwd_typed<2>(p, grid, st);
    else launch_fwd_typed<1>(p, grid, st);
  }
  return hipGetLastError() == hipSuccess ? DSQG_OK : DSQG_EHIP;
}

}  // namespace
}  // namespace dsqg

using namespace dsqg;

extern "C" int dsqg_pool_gate_workspace_size(int32_t B, int32_t N, int32_t C, int backward,
                                             size_t* bytes) {
  if (!bytes) return DSQG_EINVAL;
  const int rc = pool_shape_ok(B, N, C);
  if (rc != DSQG_OK) return rc;
  *bytes = pool_workspace(B, N, C, backward != 0);
  return DSQG_OK;
}

extern "C" int dsqg_pool_gate_fwd(const dsqg_pool_gate_fwd_args* a, dsqg_stream_t stream) {
  if (!a) return DSQG_EINVAL;
  int rc = pool_shape_ok(a->B, a->N, a->C);
  if (rc != DSQG_OK) return rc;
  if (!pool_dtype_ok(a->x_dtype) || !pool_dtype_ok(a->gate_dtype) || !pool_dtype_ok(a->out_dtype))
    return DSQG_EINVAL;
  if ((long long)a->B * a->N == 0) return DSQG_OK;
  if ((rc = pool_tensor_check(a->x, a->x_stride, a->x_dtype, a->N, a->C)) != DSQG_OK ||
      (rc = pool_tensor_check(a->gate_pre, a->gate_stride, a->gate_dtype, a->N, a->C)) != DSQG_OK ||
      (rc = pool_tensor_check(a->out, a->out_stride, a->out_dtype, a->N, a->C)) != DSQG_OK)
    return rc;
  PoolParams p = {};
  p.x = a->x; p.xs_b = a->x_stride[0]; p.xs_n = a->x_stride[1];
  p.g = a->gate_pre; p.gs_b = a->gate_stride[0]; p.gs_n = a->gate_stride[1];
  p.out = a->out; p.os_b = a->out_stride[0]; p.os_n = a->out_stride[1];
  p.B = a->B; p.N = a->N; p.C = a->C;
  p.xdt = a->x_dtype; p.gdt = a->gate_dtype; p.odt = a->out_dtype; p.ydt = a->out_dtype;
  return run_pool(p, false, a->workspace, a->workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int dsqg_pool_gate_bwd(const dsqg_pool_gate_bwd_args* a, dsqg_stream_t stream) {
  if (!a) return DSQG_EINVAL;
  int rc = pool_shape_ok(a->B, a->N, a->C);
  if (rc != DSQG_OK) return rc;
  if (!pool_dtype_ok(a->x_dtype) || !pool_dtype_ok(a->gate_dtype) || !pool_dtype_ok(a->dout_dtype))
    return DSQG_EINVAL;
  if ((long long)a->B * a->N == 0 || (!a->dx && !a->dgate_pre)) return DSQG_OK;
  if ((rc = pool_tensor_check(a->x, a->x_stride, a->x_dtype, a->N, a->C)) != DSQG_OK ||
      (rc = pool_tensor_check(a->gate_pre, a->gate_stride, a->gate_dtype, a->N, a->C)) != DSQG_OK ||
      (rc = pool_tensor_check(a->dout, a->dout_stride, a->dout_dtype, a->N, a->C)) != DSQG_OK ||
      (a->dx && (rc = pool_tensor_check(a->dx, a->dx_stride, a->x_dtype, a->N, a->C)) != DSQG_OK) ||
      (a->dgate_pre &&
       (rc = pool_tensor_check(a->dgate_pre, a->dgate_stride, a->gate_dtype, a->N, a->C)) != DSQG_OK))
    return rc;
  PoolParams p = {};
  p.x = a->x; p.xs_b = a->x_stride[0]; p.xs_n = a->x_stride[1];
  p.g = a->gate_pre; p.gs_b = a->gate_stride[0]; p.gs_n = a->gate_stride[1];
  p.dy = a->dout; p.ys_b = a->dout_stride[0]; p.ys_n = a->dout_stride[1];
  p.dx = a->dx; p.dxs_b = a->dx ? a->dx_stride[0] : 0; p.dxs_n = a->dx ? a->dx_stride[1] : p.C;
  p.dg = a->dgate_pre;
  p.dgs_b = a->dgate_pre ? a->dgate_stride[0] : 0; p.dgs_n = a->dgate_pre ? a->dgate_stride[1] : p.C;
  p.B = a->B; p.N = a->N; p.C = a->C;
  p.xdt = a->x_dtype; p.gdt = a->gate_dtype; p.ydt = a->dout_dtype; p.odt = a->dout_dtype;
  return run_pool(p, true, a->workspace, a->workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}
