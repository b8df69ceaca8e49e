// Parameter-gradient reduction (dbias, dscore_gain, dif_gain, dscale_embed's final stage), one
// wave per output element: shared by bwd_reduce_kernel (dsqg_bwd.hip) and the extra workgroups
// of the bf16 dk/dv launch (dsqg_bwd_dkdv_mfma.hip), which run it next to the dk/dv tiles.
#pragma once

#include "dsqg_common.hpp"

namespace dsqg {

// One wave per parameter-gradient element: lane l sums partials l, l+64, ... in order, then a
// fixed xor-tree combines the lanes, so the result is the same on every run.
__device__ __forceinline__ float wave_sum_fixed(float x) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) x += __shfl_xor(x, s, 64);
  return x;
}

__device__ __forceinline__ void reduce_params_wave(const ReduceParams& r, int t, int lane) {
  const int JH = r.J * r.H;
  const int per_h = r.B * r.n_chunks;  // partials per head, ordered (batch group, chunk)
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

// Waves needed for every output of r (an upper bound; surplus waves return at once).
inline long long reduce_params_waves(const ReduceParams& r) {
  return 2LL * r.J * r.H + r.H + (long long)r.J * r.D;
}

}  // namespace dsqg
