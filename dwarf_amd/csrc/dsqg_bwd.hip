// DSQG backward, launch 3 and the backward driver.
//
// bwd_reduce_kernel sums the per-workgroup parameter-gradient partials written by launch 1
// (dsqg_bwd_dq.hip) in a fixed order, so dpos_bias / dscale_embed / dscore_gain / dif_gain are
// deterministic.  The reference accumulates dpb and dse with tl.atomic_add
// (kernels/dsqg_attention_v3.py:265-271), whose summation order varies run to run.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"

namespace dsqg {

// One thread per parameter-gradient element; each sums its partials in a fixed order.
__global__ __launch_bounds__(kBlock) void bwd_reduce_kernel(ReduceParams r) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  const int JH = r.J * r.H;
  const int per_h = r.B * r.n_chunks;
  int t = i;
  if (t < JH) {  // dpos_bias[j,h]
    const int j = t / r.H, h = t - j * r.H;
    float s = 0.f;
    for (int bb = 0; bb < r.B; ++bb)
      for (int c = 0; c < r.n_chunks; ++c)
        s += r.part_bias[((long long)(bb * r.H + h) * r.n_chunks + c) * r.J + j];
    r.dpos_bias[t] = s;
    return;
  }
  t -= JH;
  if (r.dscore_gain) {
    if (t < JH) {  // dscore_gain[h,j]
      const int h = t / r.J, j = t - h * r.J;
      float s = 0.f;
      for (int bb = 0; bb < r.B; ++bb)
        for (int c = 0; c < r.n_chunks; ++c)
          s += r.part_gain[((long long)(bb * r.H + h) * r.n_chunks + c) * r.J + j];
      r.dscore_gain[t] = s;
      return;
    }
    t -= JH;
  }
  if (r.dif_gain) {
    if (t < r.H) {
      float s = 0.f;
      for (int bb = 0; bb < r.B; ++bb)
        for (int c = 0; c < r.n_chunks; ++c)
          s += r.part_if[(long long)(bb * r.H + t) * r.n_chunks + c];
      r.dif_gain[t] = s;
      return;
    }
    t -= r.H;
  }
  if (r.dscale_embed && t < r.J * r.D) {
    const long long nb = (long long)r.B * r.H * r.n_chunks;
    const long long stride = (long long)r.J * r.D;
    float s = 0.f;
    for (long long blk = 0; blk < nb; ++blk) s += r.part_se[blk * stride + t];
    r.dscale_embed[t] = s;
  }
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
  const int QPB = bwd_mfma_supported(p, D, dtype) ? 64 : kBlock / (D / 8);
  const int KPB = kBlock / (D / 8);  // dk/dv kernel rows per workgroup
  p.n_tiles = (p.N + QPB - 1) / QPB;
  p.n_tiles_kv = (p.N + KPB - 1) / KPB;
  const long long work = (long long)p.B * p.H * p.n_tiles;
  const long long target = se_grad ? 1024 : 4096;
  int tpb = (int)((work + target - 1) / target);
  if (tpb < 1) tpb = 1;
  if (tpb > p.n_tiles) tpb = p.n_tiles > 0 ? p.n_tiles : 1;
  p.tiles_per_block = tpb;
  p.n_chunks = p.n_tiles > 0 ? (p.n_tiles + tpb - 1) / tpb : 0;
}

hipError_t launch_bwd_reduce(const ReduceParams& r, hipStream_t st) {
  const long long total = 2LL * r.J * r.H + r.H + (long long)r.J * r.D;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(bwd_reduce_kernel, dim3((unsigned)((total + kBlock - 1) / kBlock)), dim3(kBlock), 0, st, r);
  return hipGetLastError();
}

}  // namespace dsqg
