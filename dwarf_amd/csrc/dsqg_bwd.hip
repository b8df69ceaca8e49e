// DSQG backward, launch 3 and the backward driver.
//
// bwd_reduce_kernel sums the per-workgroup parameter-gradient partials written by launch 1
// (dsqg_bwd_dq.hip / dsqg_bwd_dq_mfma.hip) in a fixed order, so dpos_bias / dscale_embed / dscore_gain / dif_gain are
// deterministic.  The reference accumulates dpb and dse with tl.atomic_add
// (kernels/dsqg_attention_v3.py:265-271), whose summation order varies run to run.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"

namespace dsqg {

// One wave per parameter-gradient element: lane l sums partials l, l+64, ... in order, then a
// fixed xor-tree combines the lanes, so the result is the same on every run.
__device__ __forceinline__ float wave_sum_fixed(float x) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) x += __shfl_xor(x, s, 64);
  return x;
}

__global__ __launch_bounds__(kBlock) void bwd_reduce_kernel(ReduceParams r) {
  const int lane = threadIdx.x & 63;
  int t = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  const int JH = r.J * r.H;
  const int per_h = r.B * r.n_chunks;  // partials per head, ordered (b, chunk)
  if (t < JH) {  // dpos_bias[j,h]
    const int j = t / r.H, h = t - j * r.H;
    float s = 0.f;
    for (int k = lane; k < per_h; k += 64) {
      const int bb = k / r.n_chunks, c = k - bb * r.n_chunks;
      s += r.part_bias[((long long)(bb * r.H + h) * r.n_chunks + c) * r.J + j];
    }
    s = wave_sum_fixed(s);
    if (lane == 0) r.dpos_bias[t] = s;
    return;
  }
  t -= JH;
  if (r.dscore_gain) {
    if (t < JH) {  // dscore_gain[h,j]
      const int h = t / r.J, j = t - h * r.J;
      float s = 0.f;
      for (int k = lane; k < per_h; k += 64) {
        const int bb = k / r.n_chunks, c = k - bb * r.n_chunks;
        s += r.part_gain[((long long)(bb * r.H + h) * r.n_chunks + c) * r.J + j];
      }
      s = wave_sum_fixed(s);
      if (lane == 0) r.dscore_gain[t] = s;
      return;
    }
    t -= JH;
  }
  if (r.dif_gain) {
    if (t < r.H) {
      float s = 0.f;
      for (int k = lane; k < per_h; k += 64) {
        const int bb = k / r.n_chunks, c = k - bb * r.n_chunks;
        s += r.part_if[(long long)(bb * r.H + t) * r.n_chunks + c];
      }
      s = wave_sum_fixed(s);
      if (lane == 0) r.dif_gain[t] = s;
      return;
    }
    t -= r.H;
  }
  if (r.dscale_embed && t < r.J * r.D) {
    const long long stride = (long long)r.J * r.D;
    float s = 0.f;
    for (int k = lane; k < r.se_slices; k += 64) s += r.se_stage[k * stride + t];
    s = wave_sum_fixed(s);
    if (lane == 0) r.dscale_embed[t] = s;
  }
}

// First stage of the dscale_embed sum: workgroup (x, y) sums, for 256 consecutive elements of
// [J*D], the partials of workgroups [y*se_per, (y+1)*se_per) in order.  A partial row is read
// in 1 KB runs (one float per lane, consecutive elements), not as one float per partial row
// per lane; the final per-element sum then reads only se_slices values.
__global__ __launch_bounds__(kBlock) void bwd_reduce_se_stage_kernel(ReduceParams r) {
  const long long JD = (long long)r.J * r.D;
  const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (t >= JD) return;
  const long long nb = (long long)r.B * r.H * r.n_chunks;
  const long long b0 = (long long)blockIdx.y * r.se_per;
  const long long b1 = b0 + r.se_per < nb ? b0 + r.se_per : nb;
  const float* src = r.part_se + t;
  float acc = 0.f;
#pragma unroll 8
  for (long long blk = b0; blk < b1; ++blk) acc += src[blk * JD];
  r.se_stage[blockIdx.y * JD + t] = acc;
}

bool bwd_mfma_supported(const BwdParams& p, int D, int dtype) {
  if (dtype != 1) return false;
  long long rs = p.qs.n, rmin = p.qs.n;
  const long long all[4] = {p.qs.n, p.ks.n, p.vs.n, p.dos.n};
  for (long long x : all) { rs = x > rs ? x : rs; rmin = x < rmin ? x : rmin; }
  const long long span = ((long long)p.N + p.taps.maxd + 64) * rs * 2;
  return (D == 32 || D == 64 || D == 128) && p.taps.J - p.taps.W - 1 <= kMaxSparse &&
         rmin >= D && span < (1LL << 31);
}

void bwd_plan(BwdParams& p, int D, int dtype, bool se_grad) {
  const bool mfma = bwd_mfma_supported(p, D, dtype);
  const int QPB = mfma ? 64 : kBlock / (D / 8);  // dq rows per tile
  const int KPB = mfma ? 64 : kBlock / (D / 8);  // dk/dv rows per workgroup
  p.n_tiles = (p.N + QPB - 1) / QPB;
  p.n_tiles_kv = (p.N + KPB - 1) / KPB;
  const long long work = (long long)p.B * p.H * p.n_tiles;
  // Several tiles per workgroup only to bound the [J, D] dscale_embed partials; the dbias / dg /
  // da partial rows are small next to a tile's loads, so otherwise one tile per workgroup (the
  // MFMA kernel's single-tile form then keeps no per-lane addresses across tiles).
  const long long target = se_grad ? 2048 : work;
  int tpb = (int)((work + target - 1) / (target > 0 ? target : 1));
  if (tpb < 1) tpb = 1;
  if (tpb > p.n_tiles) tpb = p.n_tiles > 0 ? p.n_tiles : 1;
  p.tiles_per_block = tpb;
  p.n_chunks = p.n_tiles > 0 ? (p.n_tiles + tpb - 1) / tpb : 0;
}

hipError_t launch_bwd_reduce(const ReduceParams& r, hipStream_t st) {
  if (r.dscale_embed && r.se_slices > 0) {
    const long long JD = (long long)r.J * r.D;
    hipLaunchKernelGGL(bwd_reduce_se_stage_kernel, dim3((unsigned)((JD + kBlock - 1) / kBlock), (unsigned)r.se_slices),
                       dim3(kBlock), 0, st, r);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const long long total = 2LL * r.J * r.H + r.H + (long long)r.J * r.D;  // outputs (upper bound)
  if (total == 0) return hipSuccess;
  const long long waves_per_block = kBlock / 64;
  hipLaunchKernelGGL(bwd_reduce_kernel, dim3((unsigned)((total + waves_per_block - 1) / waves_per_block)),
                     dim3(kBlock), 0, st, r);
  return hipGetLastError();
}

}  // namespace dsqg
