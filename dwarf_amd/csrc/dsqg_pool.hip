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
// A workgroup is CGT channel groups (8 channels per lane, 16- or 32-byte loads) times
// RL = 256 / CGT row lanes; a row lane holds RPL consecutive rows in registers, so a chunk is
// L = RL * RPL rows.  Sums run in a fixed order: results are deterministic.
//
// Element types are per tensor (f32, bf16, f16) and uniform per launch, so the type switch at
// each load is a scalar branch.  As torch computes sigmoid in the gate's dtype, s is rounded
// to that dtype before it is used; all arithmetic is fp32.
#include "../../include/dsqg.h"
#include "dsqg_common.hpp"

namespace dsqg {
namespace {

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
  int cgt_log2;   // channel groups (8 channels each) per workgroup, as a power of two
  int nchunks, ctiles, L;
  int xdt, gdt, ydt, odt;  // element types (DSQG_F32 / DSQG_BF16 / DSQG_F16)
};

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}
__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  return (uint32_t)__builtin_bit_cast(unsigned short, (_Float16)f);
}

// Eight channels starting at element offset `off` of a tensor of element type dt.
__device__ __forceinline__ void load8(const void* base, int dt, long long off, float (&v)[8]) {
  if (dt == DSQG_F32) {
    Vec8<float>::load(static_cast<const float*>(base) + off, v);
    return;
  }
  const uint4 r = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  if (dt == DSQG_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = f16_to_f32(w[i] >> 16);
    }
  }
}

__device__ __forceinline__ void store8(void* base, int dt, long long off, const float (&v)[8]) {
  if (dt == DSQG_F32) {
    Vec8<float>::store(static_cast<float*>(base) + off, v);
    return;
  }
  uint32_t w[4];
  if (dt == DSQG_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_bf16(v[2 * i]) | (f32_to_bf16(v[2 * i + 1]) << 16);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = f32_to_f16(v[2 * i]) | (f32_to_f16(v[2 * i + 1]) << 16);
  }
  *reinterpret_cast<uint4*>(static_cast<uint16_t*>(base) + off) = make_uint4(w[0], w[1], w[2], w[3]);
}

// x rounded to element type dt.
__device__ __forceinline__ float round_to(int dt, float x) {
  if (dt == DSQG_BF16) return bf16_to_f32(f32_to_bf16(x));
  if (dt == DSQG_F16) return f16_to_f32(f32_to_f16(x));
  return x;
}

__device__ __forceinline__ float sigmoid_as(int dt, float g) {
  return round_to(dt, 1.0f / (1.0f + __expf(-g)));
}

// Lane coordinates of a pool workgroup.
struct PoolLane {
  int b, chunk, cgl, rl, RL, c;  // c: first channel of this lane; active iff c < C
  bool active;
  int row0;                      // first of this lane's RPL rows
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
  q.cgl = tid & ((1 << p.cgt_log2) - 1);
  q.rl = tid >> p.cgt_log2;
  q.RL = kBlock >> p.cgt_log2;
  q.c = ((ct << p.cgt_log2) + q.cgl) * 8;
  q.active = q.c < p.C;
  q.row0 = q.chunk * p.L + q.rl * RPL;
  return q;
}

// In-place tree sum over the RL row lanes of an LDS array laid out [RL][CGT*8]; the total for
// channel group cgl ends in row 0.  Fixed order, so the result is deterministic.
__device__ __forceinline__ void tree_sum_rows(float* s, int RL, int width, int tid) {
  for (int half = RL >> 1; half > 0; half >>= 1) {
    __syncthreads();
    for (int k = tid; k < half * width; k += kBlock) s[k] += s[k + half * width];
  }
  __syncthreads();
}

// ---- Pass 1: chunk sums of x (and, backward, of dout * s / (n+1)). -----------------------
template <int RPL, bool BWD>
__global__ __launch_bounds__(kBlock) void pool_chunk_sum_kernel(PoolParams p) {
  __shared__ float sX[kBlock * 8];
  __shared__ float sP[BWD ? kBlock * 8 : 1];
  const PoolLane q = pool_lane<RPL>(p);
  const int width = 8 << p.cgt_log2;
  float ax[8], ap[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) ax[e] = ap[e] = 0.f;
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    if (q.active && n < p.N) {
      float v[8];
      load8(p.x, p.xdt, q.b * p.xs_b + n * p.xs_n + q.c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ax[e] += v[e];
      if constexpr (BWD) {
        float gv[8], yv[8];
        load8(p.g, p.gdt, q.b * p.gs_b + n * p.gs_n + q.c, gv);
        load8(p.dy, p.ydt, q.b * p.ys_b + n * p.ys_n + q.c, yv);
        const float cnt = (float)(n + 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) ap[e] += yv[e] * sigmoid_as(p.gdt, gv[e]) / cnt;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sX[q.rl * width + q.cgl * 8 + e] = ax[e];
    if constexpr (BWD) sP[q.rl * width + q.cgl * 8 + e] = ap[e];
  }
  tree_sum_rows(sX, q.RL, width, threadIdx.x);
  if constexpr (BWD) tree_sum_rows(sP, q.RL, width, threadIdx.x);
  if (q.rl == 0 && q.active) {
    const long long o = ((long long)q.b * p.nchunks + q.chunk) * p.C + q.c;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      p.px[o + e] = sX[q.cgl * 8 + e];
      if constexpr (BWD) p.pp[o + e] = sP[q.cgl * 8 + e];
    }
  }
}

// Sum over chunks k = first, first + RL, ... < end of a [B][nchunks][C] partial array.
__device__ __forceinline__ void strided_chunk_sum(const float* part, const PoolParams& p,
                                                  const PoolLane& q, int first, int end,
                                                  float (&acc)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  if (!q.active) return;
  for (int k = first; k < end; k += q.RL) {
    float v[8];
    Vec8<float>::load(part + ((long long)q.b * p.nchunks + k) * p.C + q.c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
  }
}

// ---- Pass 2, forward: out = s * (carry + running sum) / (n+1). ----------------------------
template <int RPL>
__global__ __launch_bounds__(kBlock) void pool_fwd_scan_kernel(PoolParams p) {
  __shared__ float sCarry[kBlock * 8];  // [RL][width] strided sums of earlier chunks
  __shared__ float sLane[kBlock * 8];   // [RL][width] this chunk's row-lane sums
  const PoolLane q = pool_lane<RPL>(p);
  const int width = 8 << p.cgt_log2;
  float x[RPL][8], s[RPL][8];
  float ls[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) ls[e] = 0.f;
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    if (q.active && n < p.N) {
      float gv[8];
      load8(p.x, p.xdt, q.b * p.xs_b + n * p.xs_n + q.c, x[r]);
      load8(p.g, p.gdt, q.b * p.gs_b + n * p.gs_n + q.c, gv);
#pragma unroll
      for (int e = 0; e < 8; ++e) s[r][e] = sigmoid_as(p.gdt, gv[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[r][e] = s[r][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ls[e] += x[r][e];
  }
  float cp[8];
  strided_chunk_sum(p.px, p, q, q.rl, q.chunk, cp);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sCarry[q.rl * width + q.cgl * 8 + e] = cp[e];
    sLane[q.rl * width + q.cgl * 8 + e] = ls[e];
  }
  __syncthreads();
  float run[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) run[e] = 0.f;
  for (int k = 0; k < q.RL; ++k) {
#pragma unroll
    for (int e = 0; e < 8; ++e) run[e] += sCarry[k * width + q.cgl * 8 + e];
  }
  for (int k = 0; k < q.rl; ++k) {
#pragma unroll
    for (int e = 0; e < 8; ++e) run[e] += sLane[k * width + q.cgl * 8 + e];
  }
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    float o[8];
    const float cnt = (float)(n + 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      run[e] += x[r][e];
      o[e] = s[r][e] * (run[e] / cnt);
    }
    if (q.active && n < p.N) store8(p.out, p.odt, q.b * p.os_b + n * p.os_n + q.c, o);
  }
}

// ---- Pass 2, backward. ----------------------------------------------------------------------
template <int RPL>
__global__ __launch_bounds__(kBlock) void pool_bwd_scan_kernel(PoolParams p) {
  __shared__ float sCx[kBlock * 8];  // strided sums of x over earlier chunks
  __shared__ float sLx[kBlock * 8];  // row-lane sums of x
  __shared__ float sCp[kBlock * 8];  // strided sums of dP over later chunks
  __shared__ float sLp[kBlock * 8];  // row-lane sums of dP
  const PoolLane q = pool_lane<RPL>(p);
  const int width = 8 << p.cgt_log2;
  float x[RPL][8], s[RPL][8], y[RPL][8];
  float lx[8], lp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) lx[e] = lp[e] = 0.f;
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    if (q.active && n < p.N) {
      float gv[8];
      load8(p.x, p.xdt, q.b * p.xs_b + n * p.xs_n + q.c, x[r]);
      load8(p.g, p.gdt, q.b * p.gs_b + n * p.gs_n + q.c, gv);
      load8(p.dy, p.ydt, q.b * p.ys_b + n * p.ys_n + q.c, y[r]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s[r][e] = sigmoid_as(p.gdt, gv[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[r][e] = s[r][e] = y[r][e] = 0.f;
    }
    const float cnt = (float)(n + 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lx[e] += x[r][e];
      lp[e] += y[r][e] * s[r][e] / cnt;
    }
  }
  float cx[8], cp[8];
  strided_chunk_sum(p.px, p, q, q.rl, q.chunk, cx);
  strided_chunk_sum(p.pp, p, q, q.chunk + 1 + q.rl, p.nchunks, cp);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int o = q.rl * width + q.cgl * 8 + e;
    sCx[o] = cx[e]; sLx[o] = lx[e]; sCp[o] = cp[e]; sLp[o] = lp[e];
  }
  __syncthreads();
  float runx[8], runp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) runx[e] = runp[e] = 0.f;
  for (int k = 0; k < q.RL; ++k) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      runx[e] += sCx[k * width + q.cgl * 8 + e];
      runp[e] += sCp[k * width + q.cgl * 8 + e];
    }
  }
  for (int k = 0; k < q.rl; ++k) {
#pragma unroll
    for (int e = 0; e < 8; ++e) runx[e] += sLx[k * width + q.cgl * 8 + e];
  }
  for (int k = q.RL - 1; k > q.rl; --k) {
#pragma unroll
    for (int e = 0; e < 8; ++e) runp[e] += sLp[k * width + q.cgl * 8 + e];
  }
  // dgate_pre on the way down the rows (prefix sums of x) ...
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int n = q.row0 + r;
    const float cnt = (float)(n + 1);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      runx[e] += x[r][e];
      o[e] = y[r][e] * (runx[e] / cnt) * (s[r][e] * (1.0f - s[r][e]));
    }
    if (p.dg && q.active && n < p.N) store8(p.dg, p.gdt, q.b * p.dgs_b + n * p.dgs_n + q.c, o);
  }
  // ... and dx on the way up (suffix sums of dout * s / (n+1)).
#pragma unroll
  for (int r = RPL - 1; r >= 0; --r) {
    const int n = q.row0 + r;
    const float cnt = (float)(n + 1);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      runp[e] += y[r][e] * s[r][e] / cnt;
      o[e] = runp[e];
    }
    if (p.dx && q.active && n < p.N) store8(p.dx, p.xdt, q.b * p.dxs_b + n * p.dxs_n + q.c, o);
  }
}

// ---- Host side. ------------------------------------------------------------------------------

struct PoolPlan {
  int cgt_log2, rpl, L, nchunks, ctiles;
  long long grid;
};

// Channel groups per workgroup: the smallest power of two covering C/8, at most 64; rows per
// lane: the most (4, 2, 1) that still gives at least 1024 workgroups.
PoolPlan pool_plan(int B, int N, int C) {
  PoolPlan pl;
  const int cg = C / 8;
  pl.cgt_log2 = 0;
  while ((1 << pl.cgt_log2) < cg && pl.cgt_log2 < 6) ++pl.cgt_log2;
  pl.ctiles = (cg + (1 << pl.cgt_log2) - 1) >> pl.cgt_log2;
  const int RL = kBlock >> pl.cgt_log2;
  for (int rpl = 4; rpl >= 1; rpl >>= 1) {
    pl.rpl = rpl;
    pl.L = RL * rpl;
    pl.nchunks = (N + pl.L - 1) / pl.L;
    pl.grid = (long long)B * pl.nchunks * pl.ctiles;
    if (pl.grid >= 1024) break;
  }
  return pl;
}

bool pool_dtype_ok(int dt) { return dt == DSQG_F32 || dt == DSQG_BF16 || dt == DSQG_F16; }
size_t pool_elem(int dt) { return dt == DSQG_F32 ? 4 : 2; }
size_t align256_p(size_t x) { return (x + 255) & ~size_t(255); }

// A [B,N,C] operand: 16-byte aligned base and rows, non-negative strides.
bool pool_tensor_ok(const void* ptr, const int64_t st[2], int dt) {
  if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 15u)) return false;
  const long long es = (long long)pool_elem(dt);
  for (int i = 0; i < 2; ++i)
    if (st[i] < 0 || (st[i] * es) % 16 != 0) return false;
  return true;
}

int pool_shape_ok(int B, int N, int C) {
  if (B < 0 || N < 0 || C <= 0 || C % 8 != 0) return DSQG_EINVAL;
  if ((long long)B * N * C >= (1ll << 40)) return DSQG_EUNSUPPORTED;
  return DSQG_OK;
}

size_t pool_workspace(int B, int N, int C, bool bwd) {
  const PoolPlan pl = pool_plan(B, N, C);
  const size_t one = align256_p(sizeof(float) * (size_t)B * pl.nchunks * C);
  return bwd ? 2 * one : one;
}

template <int RPL>
void launch_pool(const PoolParams& p, bool bwd, unsigned grid, hipStream_t st) {
  if (bwd) {
    hipLaunchKernelGGL((pool_chunk_sum_kernel<RPL, true>), dim3(grid), dim3(kBlock), 0, st, p);
    hipLaunchKernelGGL((pool_bwd_scan_kernel<RPL>), dim3(grid), dim3(kBlock), 0, st, p);
  } else {
    hipLaunchKernelGGL((pool_chunk_sum_kernel<RPL, false>), dim3(grid), dim3(kBlock), 0, st, p);
    hipLaunchKernelGGL((pool_fwd_scan_kernel<RPL>), dim3(grid), dim3(kBlock), 0, st, p);
  }
}

int run_pool(PoolParams& p, bool bwd, void* ws, size_t ws_bytes, hipStream_t st) {
  const PoolPlan pl = pool_plan(p.B, p.N, p.C);
  if (pl.grid == 0) return DSQG_OK;
  if (pl.grid > 0x7fffffffll) return DSQG_EUNSUPPORTED;
  const size_t one = align256_p(sizeof(float) * (size_t)p.B * pl.nchunks * p.C);
  if (!ws || (reinterpret_cast<uintptr_t>(ws) & 255u) || ws_bytes < (bwd ? 2 * one : one))
    return DSQG_EWORKSPACE;
  p.px = static_cast<float*>(ws);
  p.pp = bwd ? reinterpret_cast<float*>(static_cast<char*>(ws) + one) : nullptr;
  p.cgt_log2 = pl.cgt_log2;
  p.nchunks = pl.nchunks;
  p.ctiles = pl.ctiles;
  p.L = pl.L;
  switch (pl.rpl) {
    case 4: launch_pool<4>(p, bwd, (unsigned)pl.grid, st); break;
    case 2: launch_pool<2>(p, bwd, (unsigned)pl.grid, st); break;
    default: launch_pool<1>(p, bwd, (unsigned)pl.grid, st); break;
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
  if (!pool_tensor_ok(a->x, a->x_stride, a->x_dtype) ||
      !pool_tensor_ok(a->gate_pre, a->gate_stride, a->gate_dtype) ||
      !pool_tensor_ok(a->out, a->out_stride, a->out_dtype))
    return DSQG_EINVAL;
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
  if (!pool_tensor_ok(a->x, a->x_stride, a->x_dtype) ||
      !pool_tensor_ok(a->gate_pre, a->gate_stride, a->gate_dtype) ||
      !pool_tensor_ok(a->dout, a->dout_stride, a->dout_dtype) ||
      (a->dx && !pool_tensor_ok(a->dx, a->dx_stride, a->x_dtype)) ||
      (a->dgate_pre && !pool_tensor_ok(a->dgate_pre, a->dgate_stride, a->gate_dtype)))
    return DSQG_EINVAL;
  PoolParams p = {};
  p.x = a->x; p.xs_b = a->x_stride[0]; p.xs_n = a->x_stride[1];
  p.g = a->gate_pre; p.gs_b = a->gate_stride[0]; p.gs_n = a->gate_stride[1];
  p.dy = a->dout; p.ys_b = a->dout_stride[0]; p.ys_n = a->dout_stride[1];
  p.dx = a->dx; p.dxs_b = a->dx_stride[0]; p.dxs_n = a->dx_stride[1];
  p.dg = a->dgate_pre; p.dgs_b = a->dgate_stride[0]; p.dgs_n = a->dgate_stride[1];
  p.B = a->B; p.N = a->N; p.C = a->C;
  p.xdt = a->x_dtype; p.gdt = a->gate_dtype; p.ydt = a->dout_dtype; p.odt = a->dout_dtype;
  return run_pool(p, true, a->workspace, a->workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}
