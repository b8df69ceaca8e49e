// DSQG ring-buffer decode step (one new token per sequence).
//
// Each sequence (b,h) keeps its last S >= max(delta)+1 keys and values in a ring [S, D]; the
// token at absolute position p lives in slot p mod S.  A step writes the new (k, v) into slot
// p mod S and attends the J taps: the new row for delta = 0 and slot (p - delta) mod S for
// delta > 0, masked when p - delta < 0.  Because delta < S, no tap slot equals the slot being
// written, so the write and the reads of one step never touch the same row.
//
// One wave64 per (b,h), four per workgroup.  Lanes form R = 64/G groups of G = D/8 lanes; in
// pass t group r handles tap j = t*R + r, so the J key rows (and then the J value rows) are
// fetched as R coalesced rows at a time with all passes' loads in flight together.  The
// softmax max/sum and the output sum across groups use cross-lane shuffles.
//
// The reference has no decode kernel (train/train_2048_condU.py:463-487 recomputes the prefix);
// the ring follows README.md:175-177.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"

namespace dsqg {

template <int R>
__device__ __forceinline__ float cross_group_max(float x, int G) {
#pragma unroll
  for (int s = 1; s < R; s <<= 1) x = fmaxf(x, __shfl_xor(x, s * G, 64));
  return x;
}
template <int R>
__device__ __forceinline__ float cross_group_sum(float x, int G) {
#pragma unroll
  for (int s = 1; s < R; s <<= 1) x += __shfl_xor(x, s * G, 64);
  return x;
}

template <typename T, int D, int JMAX, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void decode_kernel(DecodeParams p) {
  constexpr int G = D / 8;
  constexpr int R = 64 / G;
  constexpr int P = (JMAX + R - 1) / R;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const long long bh = (long long)blockIdx.x * (kBlock / 64) + wave;
  if (bh >= (long long)p.B * p.H) return;
  const int b = (int)(bh / p.H), h = (int)(bh - (long long)b * p.H);
  const int r = lane / G, g = lane - r * G;
  const int d0 = g * 8;
  const int J = p.taps.J, S = p.S;
  const float c = p.scale;
  const long long pos = p.pos[b];
  T* outrow = static_cast<T*>(p.out) + bh * D;
  if (pos < 0) {  // invalid position: NaN output, ring untouched
    if (lane < G) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __int_as_float(0x7fc00000);
      Vec8<T>::store(outrow + d0, o);
    }
    return;
  }

  const T* qrow = static_cast<const T*>(p.q) + bh * D;
  const T* knew = static_cast<const T*>(p.k_new) + bh * D;
  const T* vnew = static_cast<const T*>(p.v_new) + bh * D;
  T* kring = static_cast<T*>(p.k_ring) + bh * (long long)S * D;
  T* vring = static_cast<T*>(p.v_ring) + bh * (long long)S * D;

  float q[8];
  Vec8<T>::load(qrow + d0, q);

  float s[P];
  int slot[P];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const int j = t * R + r;
    float part = 0.f, bias = 0.f;
    bool ok = false;
    slot[t] = -1;
    if (j < J) {
      const int dl = p.taps.delta[j];
      ok = pos - dl >= 0;
      bias = p.pos_bias[j * p.H + h];
      if (ok) {
        float kx[8];
        if (dl == 0) {
          Vec8<T>::load(knew + d0, kx);
        } else {
          long long sl = (pos - dl) % S;
          slot[t] = (int)sl;
          Vec8<T>::load(kring + sl * D + d0, kx);
        }
        float pk = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) pk = fmaf(q[e], kx[e], pk);
        part = pk * (p.score_gain ? p.score_gain[h * J + j] : 1.0f);
        if constexpr (HAS_SE) {
#pragma unroll
          for (int e = 0; e < 8; ++e) part = fmaf(q[e], p.scale_embed[j * D + d0 + e], part);
        }
      }
    }
    const float tot = group_sum<G>(part);
    s[t] = ok ? fmaf(tot, c, bias) : -INFINITY;
  }

  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < P; ++t) mx = fmaxf(mx, s[t]);
  mx = cross_group_max<R>(mx, G);

  float l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const float pj = __expf(s[t] - mx);
    l += pj;
    const int j = t * R + r;
    if (j < J && s[t] != -INFINITY) {
      float vx[8];
      if (slot[t] < 0) Vec8<T>::load(vnew + d0, vx);
      else Vec8<T>::load(vring + (long long)slot[t] * D + d0, vx);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(pj, vx[e], acc[e]);
    }
  }
  l = cross_group_sum<R>(l, G);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = cross_group_sum<R>(acc[e], G);

  if (r == 0) {
    const float a = p.if_gain ? p.if_gain[h] : 1.0f;
    const float inv = a / l;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = acc[e] * inv;
    Vec8<T>::store(outrow + d0, o);
    // The new row goes into slot pos mod S (read by later steps only).
    const long long sl = pos % S;
    st16(kring + sl * D + d0, ld16(knew + d0));
    if constexpr (sizeof(T) == 4) st16(kring + sl * D + d0 + 4, ld16(knew + d0 + 4));
    st16(vring + sl * D + d0, ld16(vnew + d0));
    if constexpr (sizeof(T) == 4) st16(vring + sl * D + d0 + 4, ld16(vnew + d0 + 4));
    if (p.pos_next && h == 0 && g == 0) p.pos_next[b] = pos + 1;
  }
}

template <typename T, int D, int JMAX>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t st) {
  const long long waves = (long long)p.B * p.H;
  if (waves == 0) return hipSuccess;
  const unsigned nb = (unsigned)((waves + (kBlock / 64) - 1) / (kBlock / 64));
  if (p.scale_embed)
    hipLaunchKernelGGL((decode_kernel<T, D, JMAX, true>), dim3(nb), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL((decode_kernel<T, D, JMAX, false>), dim3(nb), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_decode_d(const DecodeParams& p, hipStream_t st) {
  return launch_decode_t<T, D, kMaxTaps>(p, st);
}

template <typename T>
static hipError_t launch_decode_dtype(const DecodeParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return launch_decode_d<T, 32>(p, st);
    case 64: return launch_decode_d<T, 64>(p, st);
    case 128: return launch_decode_d<T, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode(const DecodeParams& p, int dtype, int D, hipStream_t st) {
  return dtype == 0 ? launch_decode_dtype<float>(p, D, st) : launch_decode_dtype<bf16_t>(p, D, st);
}

}  // namespace dsqg
