// Shared device helpers and launch parameter blocks for the DSQG HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsqg {

constexpr int kMaxOffsets = 64;   // DSQG_MAX_OFFSETS (size of the offset table in the ABI)
constexpr int kMaxTaps = 48;      // offsets the kernels hold in registers (J <= 48)
constexpr int kMaxSparse = 16;    // long-range taps (beyond the dense window) of the MFMA kernels
constexpr int kMaxWindow = 32;    // largest dense window staged in LDS (delta = 0..32)
constexpr int kBlock = 256;       // threads per workgroup (4 wave64)

typedef uint16_t bf16_t;

// Lanes per row of the VALU kernels: D/8 (eight elements per lane) rounded up to a power of
// two, so that a row's lanes form an aligned DPP group; for D = 80 and 96 (16 lanes) the lanes
// past the row hold zeros and store nothing.
constexpr int lanes_per_row(int D) { return D <= 32 ? 4 : (D <= 64 ? 8 : 16); }

// ---------------------------------------------------------------------------------------
// Element conversion.  bf16 is the upper half of an IEEE binary32; float -> bf16 rounds to
// nearest-even (NaN stays a quiet NaN).
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

// Load 8 consecutive elements of a row starting at p (16-byte aligned for bf16, 32 for f32).
template <typename T> struct Vec8;

template <> struct Vec8<float> {
  __device__ __forceinline__ static void load(const float* p, float (&x)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
  __device__ __forceinline__ static void store(float* p, const float (&x)[8]) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
  }
};

template <> struct Vec8<bf16_t> {
  __device__ __forceinline__ static void load(const bf16_t* p, float (&x)[8]) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static void store(bf16_t* p, const float (&x)[8]) {
    uint4 r;
    r.x = f32_to_bf16(x[0]) | (f32_to_bf16(x[1]) << 16);
    r.y = f32_to_bf16(x[2]) | (f32_to_bf16(x[3]) << 16);
    r.z = f32_to_bf16(x[4]) | (f32_to_bf16(x[5]) << 16);
    r.w = f32_to_bf16(x[6]) | (f32_to_bf16(x[7]) << 16);
    *reinterpret_cast<uint4*>(p) = r;
  }
};

// Raw 16-byte chunk copy (8 bf16 or 4 f32), used to stage rows into LDS unchanged.
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, uint4 v) { *reinterpret_cast<uint4*>(p) = v; }
__device__ __forceinline__ uint4 zero16() { return make_uint4(0u, 0u, 0u, 0u); }

// ---------------------------------------------------------------------------------------
// Cross-lane sums inside aligned groups of G consecutive lanes (G = 1, 2, 4, 8, 16), every
// lane of the group receiving the total.  DPP: quad_perm [1,0,3,2] (lane^1), quad_perm
// [2,3,0,1] (lane^2), row_half_mirror (lane i <- 7-i inside 8; after the quad steps every lane
// holds its quad's sum, so this adds the other quad), row_mirror (lane i <- 15-i inside 16).
// ---------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, true));
}

template <int G>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group size");
  if constexpr (G >= 2) x += dpp_f32<0xb1>(x);
  if constexpr (G >= 4) x += dpp_f32<0x4e>(x);
  if constexpr (G >= 8) x += dpp_f32<0x141>(x);
  if constexpr (G >= 16) x += dpp_f32<0x140>(x);
  return x;
}

// ---------------------------------------------------------------------------------------
// XCD-aware block numbering.  The dispatcher hands workgroup i to XCD (i mod 8).  Renumber so
// that each XCD receives one contiguous range of logical blocks: all tiles of one (b,h) then
// share one XCD's L2, where the long-range taps re-read the same K/V rows.
// ---------------------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int xcd_logical_block(int bid, int nblocks) {
  const int q = nblocks / kNumXcd, r = nblocks % kNumXcd;
  const int xcd = bid % kNumXcd, slot = bid / kNumXcd;
  return xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// ---------------------------------------------------------------------------------------
// Launch parameter blocks (passed by value as kernel arguments).
// ---------------------------------------------------------------------------------------
struct Strides4 {
  long long b, h, n, d;
};

struct TapTable {
  int J;        // number of offsets
  int W;        // dense window: offsets[j] == j for j <= W (W <= kMaxWindow)
  int maxd;     // largest offset
  int delta[kMaxOffsets];
  // Offsets of the long-range taps (delta[W + 1 + t]), at fixed kernel-argument slots so the
  // kernels read them with constant offsets (batched scalar loads, no waits inside tap loops).
  int sdelta[kMaxSparse];
};

struct FwdParams {
  int B, H, N;
  int n_tiles;  // query tiles per (b,h)
  float scale;  // 1/sqrt(D)
  TapTable taps;
  const void* q; Strides4 qs;
  const void* k; Strides4 ks;
  const void* v; Strides4 vs;
  const float* pos_bias;     // [J,H]
  const float* scale_embed;  // [J,D] or null
  const float* score_gain;   // [H,J] or null
  const float* if_gain;      // [H] or null
  void* out; Strides4 os;
  float* lse;                // [B,H,N] or null
  // bf16: the long-range taps' softmax weights alpha_j (pre-gain), [B,H,NS,N] fp32 with
  // NS = J - W - 1 taps beyond the dense window, or null (not written).
  float* alpha_lr;
};

struct ReduceParams {
  int B, H, J, D, n_chunks;  // B: batch groups of the partials (BwdParams::n_bgroups)
  const float* part_bias; const float* part_se; const float* part_gain; const float* part_if;
  float* dpos_bias; float* dscale_embed; float* dscore_gain; float* dif_gain;
  // dscale_embed is summed in two stages: se_slices runs of se_per consecutive workgroup
  // partials each, summed column-wise into se_stage [se_slices][J*D], then the slices.
  float* se_stage; int se_slices, se_per;
};

struct BwdParams {
  int B, H, N;
  int n_tiles;          // query tiles per (b,h) of the dq launch
  int tiles_per_block;  // consecutive tiles of one (b,h) handled by one dq workgroup
  int n_chunks;         // dq workgroups per (b,h)
  // bf16 MFMA dq: batches handled by one workgroup (the same head and tile of each), and the
  // batch groups that gives; the parameter partials are [n_bgroups * H * n_chunks].
  int batches_per_block;
  int n_bgroups;
  int n_tiles_kv;       // key tiles per (b,h) of the dk/dv launch (one workgroup each)
  float scale;
  TapTable taps;
  const void* q; Strides4 qs;
  const void* k; Strides4 ks;
  const void* v; Strides4 vs;
  const void* dout; Strides4 dos;
  const float* lse;
  const float* alpha_lr;  // bf16: the forward's long-range weights [B,H,NS,N] (FwdParams::alpha_lr)
  const float* pos_bias;
  const float* scale_embed;
  const float* score_gain;
  const float* if_gain;
  void* dq; Strides4 dqs;
  void* dk; Strides4 dks;
  void* dv; Strides4 dvs;
  float* dpre;        // workspace [B,H,N]: D' = dOut . o (pre-gain o), fp32
  float* part_bias;   // workspace [n_bgroups*H*n_chunks][J]
  float* part_se;     // workspace [n_bgroups*H*n_chunks][J][D] or null
  float* part_gain;   // workspace [n_bgroups*H*n_chunks][J] or null
  float* part_if;     // workspace [n_bgroups*H*n_chunks] or null
  // bf16 MFMA path: the long-range taps' weights, written by dq and read by dk/dv, workspace
  // [B*H][NS][N] dwords (NS = taps beyond the dense window), for query n and tap W + 1 + t:
  // low half bf16(c g_j dS_j) (the weight of q_n in dk), high half bf16(a alpha_j) (the weight
  // of dOut_n in dv).
  float* lrw;
  // Parameter reduction run by red_blocks extra workgroups of the bf16 dk/dv launch (0: none).
  ReduceParams red;
  int red_blocks;
};


struct DecodeParams {
  int B, H, S;
  float scale;
  TapTable taps;
  const void* q; const void* k_new; const void* v_new;
  void* k_ring; void* v_ring;
  const long long* pos; long long* pos_next;
  const float* pos_bias; const float* scale_embed; const float* score_gain;
  const float* if_gain;
  void* out;
};

}  // namespace dsqg
