// DSQG ring-buffer decode step (one new token per sequence).
//
// Each sequence (b,h) keeps its last S >= max(delta)+1 keys and values in a ring [S, D]; the
// token at absolute position p lives in slot p mod S.  A step writes the new (k, v) into slot
// p mod S and attends the J taps: the new row for delta = 0 and slot (p - delta) mod S for
// delta > 0, masked when p - delta < 0.  Because delta < S, no tap slot equals the slot being
// written, so the write and the reads of one step never touch the same row.
//
// One wave64 per (b,h), four per workgroup.  Lanes form R = 64/G groups of G = D/8 lanes; in
// pass t group r handles tap j = t*R + r, so the J key and value rows are fetched as R
// coalesced rows at a time, all of them requested before any arithmetic (two dependent memory
// round trips per step: the position, then the ring rows it selects).  The softmax max/sum
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

template <typename T, int D, int JMAX, bool HAS_SE>
__global__ __launch_bounds__(kBlock) void decode_kernel(DecodeParams p) {
  constexpr int G = lanes_per_row(D);  // lanes with 8g >= D (D = 80, 96) hold zeros
  constexpr int R = 64 / G;
  constexpr int P = (JMAX + R - 1) / R;
  constexpr int E = sizeof(T);

  const int lane = threadIdx.x & 63;
  // The wave index is uniform: readfirstlane keeps (b, h), the row pointers and the ring's buffer
  // resources in scalar registers (a resource in vector registers costs every load a loop).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // One round trip for the kernel arguments before the position's: the arguments the prologue
  // needs pass through one empty asm statement that everything after it depends on, so their
  // scalar loads go out together and are waited for once (otherwise the compiler waits for B
  // and H, divides, and only then asks for the pointers).  For the same reason no wave exits
  // early: waves past the last (b,h) (B * H not a multiple of four) repeat it and store nothing.
  int nB = p.B, nH = p.H, J = p.taps.J;
  const long long* posp = p.pos;
  const void *qp = p.q, *knp = p.k_new, *vnp = p.v_new;
  const float* pbp = p.pos_bias;
  asm volatile("" : "+s"(nB), "+s"(nH), "+s"(J) : "s"(posp), "s"(qp), "s"(knp), "s"(vnp), "s"(pbp));
  const long long nbh = (long long)nB * nH;
  const long long bh_w = (long long)blockIdx.x * (kBlock / 64) + wave;
  const bool live = bh_w < nbh;
  const long long bh = live ? bh_w : nbh - 1;
  const int b = (int)bh / nH, h = (int)bh - b * nH;  // B * H < 2^31 (checked by the ABI)
  const int r = lane / G, g = lane - r * G;
  const int d0 = g * 8;
  const bool lane_ok = d0 < D;
  const int S = p.S;
  const float c = p.scale;
  const long long pos = posp[b];  // waited for at the validity test below
  T* outrow = static_cast<T*>(p.out) + bh * D;
  const T* qrow = static_cast<const T*>(qp) + bh * D;
  const T* knew = static_cast<const T*>(knp) + bh * D;
  const T* vnew = static_cast<const T*>(vnp) + bh * D;

  // Two memory round trips per step.  Everything that does not depend on the position (query,
  // new key/value row, per-tap bias, gain and scale_embed) is requested before the position is
  // waited for, and with scale_embed each pass's share of q.se_j is formed meanwhile; the ring
  // rows of the taps follow the position, all requested before the rest of the arithmetic.
  // Tap 0 (delta = 0) is the new row, already in registers; so is the row written into the ring.
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
    pbias[t] = pbp[jj * nH + h];
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

  if (pos < 0) {  // invalid position: NaN output, ring untouched, pos_next keeps it invalid
    if (live && p.pos_next && h == 0 && lane == 0) p.pos_next[b] = pos;
    if (live && lane < G && lane_ok) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __int_as_float(0x7fc00000);
      Vec8<T>::store(outrow + d0, o);
    }
    return;
  }
  if (live && p.pos_next && h == 0 && lane == 0) p.pos_next[b] = pos + 1;

  T* kring = static_cast<T*>(p.k_ring) + bh * (long long)S * D;
  T* vring = static_cast<T*>(p.v_ring) + bh * (long long)S * D;
  // Ring reads go through buffer resources over this sequence's ring: a masked tap gets an
  // offset past the end and reads zeros, so it needs no select in the weighted sum.
  const __amdgpu_buffer_rsrc_t rK = __builtin_amdgcn_make_buffer_rsrc(kring, (short)0, S * D * E, 0x00020000);
  const __amdgpu_buffer_rsrc_t rV = __builtin_amdgcn_make_buffer_rsrc(vring, (short)0, S * D * E, 0x00020000);

  // Slot of tap delta: (pos mod S) - delta, wrapped once (0 < delta < S).  The new row goes
  // into slot pos mod S now: no tap of this step reads that slot.
  const int base = (pos >> 31) == 0 ? (int)pos % S : (int)(pos % S);  // 32-bit when it fits
  if (live && r == 0 && lane_ok) {
#pragma unroll
    for (int u = 0; u < C16; ++u) {
      st16(kring + base * D + d0 + 4 * u * (E == 4), knraw[u]);
      st16(vring + base * D + d0 + 4 * u * (E == 4), vnraw[u]);
    }
  }
  uint4 kraw[P][C16], vraw[P][C16];
  bool ok[P];
#pragma unroll
  for (int t = 0; t < P; ++t) {
    const int j = t * R + r;
    const int dl = j < J ? p.taps.delta[j] : 0;
    ok[t] = j < J && pos - dl >= 0;
    if (dl > 0) {
      const int sw = base - dl;
      const unsigned off = ok[t] && lane_ok ? (unsigned)(((sw < 0 ? sw + S : sw) * D + d0) * E) : 0x80000000u;
#pragma unroll
      for (int u = 0; u < C16; ++u) {
        kraw[t][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rK, off + 16 * u, 0, 0));
        vraw[t][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rV, off + 16 * u, 0, 0));
      }
    } else {
#pragma unroll
      for (int u = 0; u < C16; ++u) { kraw[t][u] = knraw[u]; vraw[t][u] = vnraw[u]; }
    }
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

  // Masked taps have weight exp(-inf) = 0 and zero rows; taps j >= J hold the new row (finite).
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
