// DSQG ring-buffer decode step (one new token per sequence).
//
// Each sequence (b,h) keeps its last S >= max(delta)+1 keys and values in a ring [S, D]; the
// token at absolute position p lives in slot p mod S.  A step writes the new (k, v) into slot
// p mod S and attends the J taps: the new row for delta = 0 and slot (p - delta) mod S for
// delta > 0, masked when p - delta < 0.  Because delta < S, no tap slot equals the slot being
// written, so the write and the reads of one step never touch the same row.
//
// One wave64 per (b,h), four heads of one sequence per workgroup.  Lanes form R = 64/G groups of
// G = D/8 lanes; in pass t group r handles tap j = t*R + r, so the J key and value rows are
// fetched as R coalesced rows at a time, all of them requested together before any arithmetic
// (two dependent memory round trips per step: the position, then the ring rows it selects).  The softmax max/sum
// and the output sum across groups use DPP and v_permlane16/32_swap (no LDS).
//
// The reference has no decode kernel (train/train_2048_condU.py:463-487 recomputes the prefix);
// the ring follows README.md:175-177.
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"
#include "dsqg_mfma.hpp"

namespace dsqg {

// Combine the R lane groups of G = 64/R lanes (lanes l, l^G, l^2G, ...): xor 4 (G = 4 only)
// by a lane shuffle, xor 8 inside a 16-lane row by DPP row_ror:8, xor 16 / xor 32 by
// v_permlane16/32_swap.  Every lane ends with
// the total; the pairing order is the same on both lanes of each pair.
template <int R>
__device__ __forceinline__ float groups_reduce_sum(float x) {
  constexpr int G = 64 / R;
  if constexpr (G <= 4) x += __shfl_xor(x, 4, 64);                        // lane ^ 4
  if constexpr (G <= 8) x += dpp_f32<0x128>(x);                           // lane ^ 8
  if constexpr (G <= 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);                    // lane ^ 16
  }
  const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r2[0]) + __uint_as_float(r2[1]);                 // lane ^ 32
}
template <int R>
__device__ __forceinline__ float groups_reduce_max(float x) {
  constexpr int G = 64 / R;
  if constexpr (G <= 4) x = fmaxf(x, __shfl_xor(x, 4, 64));
  if constexpr (G <= 8) x = fmaxf(x, dpp_f32<0x128>(x));
  if constexpr (G <= 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
  const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r2[0]), __uint_as_float(r2[1]));
}

// Reduce-scatter of the eight per-lane output partials over the lane groups: at each level
// (lane ^ 32, lane ^ 16 by v_permlane32/16_swap, lane ^ 8 by DPP row_ror:8) a lane keeps half
// of its values and adds the partner's matching half, so one swap and one add move two values.
// For D <= 64 every lane ends with one element, index (lane >> 3) & 7 of its 8-element chunk;
// for D = 128 (four groups) with two, indices 4 (lane >> 5 & 1) + 2 (lane >> 4 & 1) + {0, 1}.
// A level whose partner lies in the same group (D = 128 at lane ^ 8) is skipped; D = 32 adds
// the remaining group bit (lane ^ 4) as a plain sum.
template <int G>
__device__ __forceinline__ void groups_scatter_sum(float (&a)[8]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[e]), __float_as_uint(a[e + 4]), false, false);
    a[e] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[e]), __float_as_uint(a[e + 2]), false, false);
    a[e] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  if constexpr (G <= 8) {
    const bool hi = (threadIdx.x & 8) != 0;
    const float keep = hi ? a[1] : a[0], send = hi ? a[0] : a[1];
    a[0] = keep + dpp_f32<0x128>(send);  // row_ror:8 = lane ^ 8 inside the 16-lane row
  }
  if constexpr (G == 4) a[0] += __shfl_xor(a[0], 4, 64);
}

// The position and the row pointers come first, as plain kernel arguments: they are preloaded
// into scalar registers at wave launch (kernel-argument preloading, gfx950), so the position's
// load is the first instruction of the wave instead of waiting for a kernel-argument round trip.
template <typename T, int D, int JMAX, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void decode_kernel(const long long* __restrict__ pos,
                                                        long long* __restrict__ pos_next,
                                                        const T* __restrict__ qp, const T* __restrict__ knp,
                                                        const T* __restrict__ vnp, T* k_ring, T* v_ring,
                                                        DecodeParams p) {
  constexpr int G = lanes_per_row(D);  // lanes with 8g >= D (D = 80, 96) hold zeros
  constexpr int R = 64 / G;
  constexpr int P = (JMAX + R - 1) / R;
  constexpr int E = sizeof(T);

  // Sequence b = blockIdx.x, heads 4 * blockIdx.y + wave: no division.  Waves past the last head
  // (H not a multiple of four) repeat it and store nothing, so that no wave exits early.
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int r = lane / G, g = lane - r * G;
  // The two loads the ring rows' addresses need go out first, before any other argument is
  // read: the position (a vector load of a uniform address, so that waiting for it does not
  // also wait for the scalar argument loads) and this lane's tap offset of each pass (from the
  // argument block, whose address every wave has at launch).
  const long long pos_v = __builtin_nontemporal_load(pos + b + opaque(0));
  int dlv[P];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const int j = t * R + r;
    dlv[t] = p.taps.delta[j < JMAX ? j : 0];  // taps j >= J are masked below
  }
  __builtin_amdgcn_sched_barrier(0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = p.H, J = p.taps.J, S = p.S;
  const int h0 = (int)blockIdx.y * (kBlock / 64) + wave;
  const bool live = h0 < H;
  const int h = live ? h0 : H - 1;
  const long long bh = (long long)b * H + h;
  const int d0 = g * 8;
  const bool lane_ok = d0 < D;
  const float c = p.scale;
  T* outrow = static_cast<T*>(p.out) + bh * D;
  const T* qrow = qp + bh * D;
  const T* knew = knp + bh * D;
  const T* vnew = vnp + bh * D;

  // Everything else that does not depend on the position is requested before it is waited
  // for: the query, the new key/value row, and per pass this lane's bias, gain and (with
  // scale_embed) its share of q.se_j.  Tap 0 (delta = 0) is the new row, already in registers;
  // so is the row written into the ring.
  constexpr int C16 = E == 4 ? 2 : 1;  // 16-byte chunks per lane (8 elements)
  uint4 qraw[C16], knraw[C16], vnraw[C16];
#pragma unroll
  for (int u = 0; u < C16; ++u) {
    qraw[u] = lane_ok ? ld16(qrow + d0 + 4 * u * (E == 4)) : zero16();
    knraw[u] = lane_ok ? ld16(knew + d0 + 4 * u * (E == 4)) : zero16();
    vnraw[u] = lane_ok ? ld16(vnew + d0 + 4 * u * (E == 4)) : zero16();
  }
  float pbias[P], pgain[P];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const int j = t * R + r;
    const int jj = j < J ? j : 0;
    pbias[t] = p.pos_bias[jj * H + h];
    pgain[t] = p.score_gain ? p.score_gain[h * J + jj] : 1.0f;
  }
  float q[8];
  Vec8<T>::load(reinterpret_cast<const T*>(qraw), q);
  float sed[P];  // this lane's share of q.se_j for the pass-t tap (summed over the row with q.k)
  if constexpr (HAS_SE) {
    float sev[P][8];
#pragma unroll
    for (int t = 0; t < P; ++t) {
      const int j = t * R + r;
      const int jj = j < J ? j : 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) sev[t][e] = lane_ok ? p.scale_embed[jj * D + d0 + e] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < P; ++t) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(q[e], sev[t][e], acc);
      sed[t] = acc;
    }
  }

  // The uniform position in scalar registers (the low half zero-extended).
  const long long pos_b = (long long)(unsigned)__builtin_amdgcn_readfirstlane((int)pos_v) |
                          ((long long)__builtin_amdgcn_readfirstlane((int)(pos_v >> 32)) << 32);
  if (pos_b < 0) {  // invalid position: NaN output, ring untouched, pos_next keeps it invalid
    if (live && pos_next && h == 0 && lane == 0) pos_next[b] = pos_b;
    if (live && lane < G && lane_ok) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __int_as_float(0x7fc00000);
      Vec8<T>::store(outrow + d0, o);
    }
    return;
  }
  if (live && pos_next && h == 0 && lane == 0) pos_next[b] = pos_b + 1;

  T* kring = k_ring + bh * (long long)S * D;
  T* vring = v_ring + bh * (long long)S * D;
  // Ring reads go through buffer resources over this sequence's ring: a masked tap (and tap 0,
  // whose row is the new one) gets an offset past the end and reads zeros, so the loads need no
  // branch and all of them are in flight together.
  const __amdgpu_buffer_rsrc_t rK = __builtin_amdgcn_make_buffer_rsrc(kring, (short)0, S * D * E, 0x00020000);
  const __amdgpu_buffer_rsrc_t rV = __builtin_amdgcn_make_buffer_rsrc(vring, (short)0, S * D * E, 0x00020000);

  // Slot of tap delta: (pos mod S) - delta, wrapped once (0 < delta < S).
  const int base = (pos_b >> 31) == 0 ? (int)pos_b % S : (int)(pos_b % S);  // 32-bit when it fits
  uint4 kraw[P][C16], vraw[P][C16];
  bool ok[P];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const int j = t * R + r;
    const int dl = dlv[t];
    ok[t] = j < J && pos_b - dl >= 0;
    const int sw = base - dl;
    const unsigned off = ok[t] && dl > 0 && lane_ok ? (unsigned)(((sw < 0 ? sw + S : sw) * D + d0) * E)
                                                   : 0x80000000u;
#pragma unroll
    for (int u = 0; u < C16; ++u) {
      kraw[t][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rK, off + 16 * u, 0, 0));
      vraw[t][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rV, off + 16 * u, 0, 0));
    }
  }
  // The new row goes into slot pos mod S once every ring load is in flight (no tap of this step
  // reads that slot, and waiting for the new row first would hold the ring loads back).
  if (live && r == 0 && lane_ok) {
#pragma unroll
    for (int u = 0; u < C16; ++u) {
      st16(kring + base * D + d0 + 4 * u * (E == 4), knraw[u]);
      st16(vring + base * D + d0 + 4 * u * (E == 4), vnraw[u]);
    }
  }
  // Tap 0 (group 0 of pass 0) takes the new row.
  if (r == 0) {
#pragma unroll
    for (int u = 0; u < C16; ++u) { kraw[0][u] = knraw[u]; vraw[0][u] = vnraw[u]; }
  }

  float s[P];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    float pk = 0.f;
    if constexpr (E == 2) {
      pk = dot8_bf16(qraw[0], kraw[t][0], 0.f);
    } else {
      float kx[8];
      Vec8<T>::load(reinterpret_cast<const T*>(kraw[t]), kx);
#pragma unroll
      for (int e = 0; e < 8; ++e) pk = fmaf(q[e], kx[e], pk);
    }
    float part = pk * pgain[t];
    if constexpr (HAS_SE) part += sed[t];
    const float tot = group_sum<G>(part);
    s[t] = ok[t] ? fmaf(tot, c, pbias[t]) : -INFINITY;
  }

  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < P; ++t) mx = fmaxf(mx, s[t]);
  mx = groups_reduce_max<R>(mx);

  // Masked taps have weight exp(-inf) = 0 and zero rows.
  float l = 0.f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const float pj = __expf(s[t] - mx);
    l += pj;
    float vx[8];
    Vec8<T>::load(reinterpret_cast<const T*>(vraw[t]), vx);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(pj, vx[e], acc[e]);
  }
  l = groups_reduce_sum<R>(l);
  groups_scatter_sum<G>(acc);

  const float a = p.if_gain ? p.if_gain[h] : 1.0f;
  const float inv = a / l;
  if constexpr (G == 16) {  // two elements per lane: 4 (lane>>5 & 1) + 2 (lane>>4 & 1) + {0,1}
    const int e0 = 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1);
    if (live && lane_ok) {
      if constexpr (E == 2) {
        *reinterpret_cast<unsigned*>(outrow + d0 + e0) =
            f32_to_bf16(acc[0] * inv) | (f32_to_bf16(acc[1] * inv) << 16);
      } else {
        *reinterpret_cast<float2*>(outrow + d0 + e0) = make_float2(acc[0] * inv, acc[1] * inv);
      }
    }
  } else if (live && (G == 8 || (r & 1) == 0)) {  // one element per lane (D = 32: both lanes of a pair hold it)
    const int e0 = (lane >> 3) & 7;
    if constexpr (E == 2) {
      outrow[d0 + e0] = (T)f32_to_bf16(acc[0] * inv);
    } else {
      outrow[d0 + e0] = acc[0] * inv;
    }
  }
}

template <typename T, int D, int JMAX>
static hipError_t launch_decode_t(const DecodeParams& p, hipStream_t st) {
  if ((long long)p.B * p.H == 0) return hipSuccess;
  const dim3 grid((unsigned)p.B, (unsigned)((p.H + (kBlock / 64) - 1) / (kBlock / 64)));
  const long long* pos = p.pos;
  const T* q = static_cast<const T*>(p.q);
  const T* kn = static_cast<const T*>(p.k_new);
  const T* vn = static_cast<const T*>(p.v_new);
  T* kr = static_cast<T*>(p.k_ring);
  T* vr = static_cast<T*>(p.v_ring);
  if (p.scale_embed)
    hipLaunchKernelGGL((decode_kernel<T, D, JMAX, true>), grid, dim3(kBlock), 0, st, pos, p.pos_next, q, kn, vn, kr, vr, p);
  else
    hipLaunchKernelGGL((decode_kernel<T, D, JMAX, false>), grid, dim3(kBlock), 0, st, pos, p.pos_next, q, kn, vn, kr, vr, p);
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
    case 80: return launch_decode_d<T, 80>(p, st);
    case 96: return launch_decode_d<T, 96>(p, st);
    case 128: return launch_decode_d<T, 128>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode(const DecodeParams& p, int dtype, int D, hipStream_t st) {
  return dtype == 0 ? launch_decode_dtype<float>(p, D, st) : launch_decode_dtype<bf16_t>(p, D, st);
}

}  // namespace dsqg
