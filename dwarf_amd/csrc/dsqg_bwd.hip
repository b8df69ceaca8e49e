// DSQG backward, launch 3 and the backward driver.
//
// bwd_reduce_kernel sums the per-workgroup parameter-gradient partials written by launch 1
// (dsqg_bwd_dq.hip / dsqg_bwd_dq_mfma.hip) in a fixed order, so dpos_bias / dscale_embed / dscore_gain / dif_gain are
// deterministic.  The reference accumulates dpb and dse with tl.atomic_add
// (kernels/dsqg_attention_v3.py:265-271), whose summation order varies run to run.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_reduce.hpp"

namespace dsqg {

__global__ __launch_bounds__(kBlock) void bwd_reduce_kernel(ReduceParams r) {
  reduce_params_wave(r, blockIdx.x * (kBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), threadIdx.x & 63);
}

// First stage of the dscale_embed sum: workgroup (x, y) sums, for 1024 consecutive elements of
// [J*D] (four per thread, one 16-byte load per partial row), the partials of workgroups
// [y*se_per, (y+1)*se_per) in order.  Each wave reads 1 KB runs; the final per-element sum then
// reads only se_slices values.
__global__ __launch_bounds__(kBlock) void bwd_reduce_se_stage_kernel(ReduceParams r) {
  const long long JD4 = (long long)r.J * r.D / 4;  // D is a multiple of 16
  const long long t = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (t >= JD4) return;
  const long long nb = (long long)r.B * r.H * r.n_chunks;
  const long long b0 = (long long)blockIdx.y * r.se_per;
  const long long b1 = b0 + r.se_per < nb ? b0 + r.se_per : nb;
  const float4* src = reinterpret_cast<const float4*>(r.part_se) + t;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (long long blk = b0; blk < b1; ++blk) {
    const float4 x = src[blk * JD4];
    acc.x += x.x; acc.y += x.y; acc.z += x.z; acc.w += x.w;
  }
  reinterpret_cast<float4*>(r.se_stage)[blockIdx.y * JD4 + t] = acc;
}

bool bwd_mfma_supported(const BwdParams& p, int D, int dtype) {
  if (dtype != 1) return false;
  long long rs = p.qs.n, rmin = p.qs.n;
  const long long all[4] = {p.qs.n, p.ks.n, p.vs.n, p.dos.n};
  for (long long x : all) { rs = x > rs ? x : rs; rmin = x < rmin ? x : rmin; }
  const long long span = ((long long)p.N + p.taps.maxd + 64) * rs * 2;
  return (D == 32 || D == 64 || D == 80 || D == 96 || D == 128) && p.taps.J - p.taps.W - 1 <= kMaxSparse &&
         rmin >= D && span < (1LL << 31);
}

void bwd_plan(BwdParams& p, int D, int dtype, bool se) {
  const bool mfma = bwd_mfma_supported(p, D, dtype);
  const int QPB = mfma ? 64 : kBlock / lanes_per_row(D);  // dq rows per tile
  const int KPB = mfma ? 64 : kBlock / lanes_per_row(D);  // dk/dv rows per workgroup
  p.n_tiles = (p.N + QPB - 1) / QPB;
  p.n_tiles_kv = (p.N + KPB - 1) / KPB;
  // One tile per workgroup: the partial rows (J floats) are small next to a tile's loads, and the
  // single-tile form keeps no per-lane addresses across tiles.  The bf16 dq with scale_embed
  // takes the same head and tile of four batches per workgroup instead: its [J x D] fp32 dse
  // partial is as large as a tile's dS, so one per tile costs as many bytes again as the tile's
  // dq (written, then read back by the reduction); one per four tiles cuts them to a quarter.
  // (Four consecutive tiles of one (b,h) instead put every tile of four times as many (b,h)
  // slices in flight at once, which overflowed L2: 143 MB more L2-miss reads per launch.)
  // dse sums over every b and h, dbias / dg / da over b, so a partial may span batches.
  p.tiles_per_block = 1;
  p.n_chunks = p.n_tiles;
  p.batches_per_block = (mfma && se) ? (p.B < 4 ? (p.B > 0 ? p.B : 1) : 4) : 1;
  p.n_bgroups = (p.B + p.batches_per_block - 1) / p.batches_per_block;
}

hipError_t launch_bwd_reduce_se_stage(const ReduceParams& r, hipStream_t st) {
  if (r.dscale_embed && r.se_slices > 0) {
    const long long JD4 = (long long)r.J * r.D / 4;
    hipLaunchKernelGGL(bwd_reduce_se_stage_kernel, dim3((unsigned)((JD4 + kBlock - 1) / kBlock), (unsigned)r.se_slices),
                       dim3(kBlock), 0, st, r);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_bwd_reduce(const ReduceParams& r, hipStream_t st) {
  const hipError_t e = launch_bwd_reduce_se_stage(r, st);
  if (e != hipSuccess) return e;
  return launch_bwd_reduce_final(r, st);
}

hipError_t launch_bwd_reduce_final(const ReduceParams& r, hipStream_t st) {
  const long long total = reduce_params_waves(r);
  if (total == 0) return hipSuccess;
  const long long waves_per_block = kBlock / 64;
  hipLaunchKernelGGL(bwd_reduce_kernel, dim3((unsigned)((total + waves_per_block - 1) / waves_per_block)),
                     dim3(kBlock), 0, st, r);
  return hipGetLastError();
}

}  // namespace dsqg
