// MFMA and LDS-transpose helpers for the gfx950 bf16 DSQG kernels.
//
// Lane layouts (wave64, measured on MI355X):
//  * v_mfma_f32_16x16x32_bf16: A lane l holds row l%16, k = 8*(l/16) .. +7; B lane l holds
//    column l%16, k = 8*(l/16) .. +7; C/D lane l holds column l%16, rows 4*(l/16) + r, r=0..3.
//  * v_mfma_f32_16x16x16_bf16: the same with k = 4*(l/16) .. +3.
//  * ds_read_tr16_b64: inside each group of 16 lanes, if lane j addresses the 4-element row
//    M[j][0..3], lane i receives M[4e + i/4][i%4] for e = 0..3.  So with a row-major [row][col]
//    bf16 tile in LDS, lane i of group g addressing  &T[r0 + 4g + i/4][c0 + 4*(i%4)]  receives
//    T[r0 + 4g + e][c0 + i], e = 0..3: the transposed 16x16x16 operand (row = column c0+i of
//    T, k = rows r0+4g .. +3) with no shuffles.
#pragma once

#include "dsqg_common.hpp"

namespace dsqg {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t mfma_16x16x16(s16x4_t a, s16x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ s16x4_t lds_read_tr16(const bf16_t* p) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Two floats -> one dword of two bf16 (a in the low half), round to nearest even: a vector
// conversion, so one v_cvt_pk_bf16_f32 takes both (element-wise conversions each take one and
// a v_perm_b32 pairs them).
__device__ __forceinline__ unsigned cvt_pk_bf16(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// Four floats -> packed bf16 operand (round to nearest even).
__device__ __forceinline__ s16x4_t pack_bf16x4(float a, float b, float c, float d) {
  return __builtin_bit_cast(s16x4_t, make_uint2(cvt_pk_bf16(a, b), cvt_pk_bf16(c, d)));
}

__device__ __forceinline__ uint2 pack_bf16x4_u2(float a, float b, float c, float d) {
  return __builtin_bit_cast(uint2, pack_bf16x4(a, b, c, d));
}

__device__ __forceinline__ f32x4_t zero4() { return f32x4_t{0.f, 0.f, 0.f, 0.f}; }

// acc + a . b over eight bf16 pairs (v_dot2_f32_bf16: exact products, fp32 accumulation).
__device__ __forceinline__ float dot8_bf16(uint4 a, uint4 b, float acc) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x), __builtin_bit_cast(bf16x2_t, b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y), __builtin_bit_cast(bf16x2_t, b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z), __builtin_bit_cast(bf16x2_t, b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w), __builtin_bit_cast(bf16x2_t, b.w), acc, false);
  return acc;
}

// acc + a.x b.x + a.y b.y for two bf16 pairs given as dword bit patterns (v_dot2_f32_bf16:
// exact products, fp32 sum).  With b = (w, 0) or (0, w) it adds w times one element of a.
__device__ __forceinline__ float dot2_bf16_bits(unsigned a, unsigned b, float acc) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc, false);
}

// Head-dim geometry of the bf16 MFMA kernels; D is a multiple of 16 in [32, 128].
//  * The MFMA K-steps cover DP = D rounded up to 32.  For D = 80 the 16 extra columns are zero
//    in every operand (loaded as zeros, staged as zeros).
//  * A row is CPR = D/8 16-byte chunks.  The row-chunk layout (below) gives a row CPRP lanes
//    (a power of two, so that DPP sums run over aligned lane groups) of CPL chunks each: rows of
//    4, 8 or 16 chunks take that many lanes with one chunk each; rows of 10 or 12 chunks
//    (D = 80, 96) take four lanes with three chunks each.  Chunks >= CPR carry zeros and store
//    nothing.
template <int D>
struct Geo {
  static_assert(D % 16 == 0 && D >= 32 && D <= 128, "head dim");
  static constexpr int DP = (D + 31) / 32 * 32;
  static constexpr int KS = DP / 32;        // 16x16x32 K-steps over the head dim
  static constexpr int DB = D / 16;         // 16-wide head-dim blocks of an output
  static constexpr int CPR = D / 8;         // 16-byte chunks of a row
  static constexpr int CPS = DP / 8;        // ... of a staged (padded) LDS row
  static constexpr int CPRP = (CPR & (CPR - 1)) == 0 ? CPR : 4;  // lanes per row
  static constexpr int CPL = (CPR + CPRP - 1) / CPRP;          // chunks per lane and row
  static constexpr int CHW = CPL * 16 * CPRP / 64;  // chunks per lane of a wave's 16-row block
  static constexpr int RV = DP + 8;         // LDS row stride (elements)
};

// Row-chunk layout of a wave's 16-row block of a [rows][D] bf16 matrix: load u (0 .. CHW-1)
// gives lane l chunk l % CPRP + CPRP (u % CPL) of row l / CPRP + (64 / CPRP) (u / CPL).  With
// one chunk per lane and row (CPL = 1) that is chunk (l + 64u) % CPRP of row (l + 64u) / CPRP,
// eight (D = 64) consecutive lanes reading one whole 128-byte row; at D = 96 load u reads
// 64-byte piece u of all 16 rows, four lanes each.  Either way each group of four consecutive
// lanes reads 64 contiguous bytes, which the vector L1 serves at close to four times the rate of
// the MFMA operand order (16 rows x 16 bytes per 16 lanes), where every group of four lanes
// touches four different cache lines; on this GPU the D = 96 order gathers 16-row blocks from L2
// as fast as the D = 64 one, and a fifth faster than 16 lanes per row with four idle.
// Lane l's CPL loads u = rg CPL .. rg CPL + CPL - 1 are chunks of one row (row group rg): a sum
// across a row adds those CPL partials in the lane, then the CPRP lanes (group_sum).
template <int D>
__device__ __forceinline__ int rc_row(int l, int u) {
  return l / Geo<D>::CPRP + (64 / Geo<D>::CPRP) * (u / Geo<D>::CPL);
}
template <int D>
__device__ __forceinline__ int rc_chunk(int l, int u) {
  return l % Geo<D>::CPRP + Geo<D>::CPRP * (u % Geo<D>::CPL);
}
template <int D>
__device__ __forceinline__ bool rc_valid(int l, int u) { return rc_chunk<D>(l, u) < Geo<D>::CPR; }

// An element offset that a slice's buffer resource turns into zeros when added to any row
// offset a kernel forms: with (N + max offset + 64) * rs * 2 < 2^31 (checked at launch), every
// row offset r * rs lies in (-2^30, 2^30), so r * rs + kNoElem is past the slice's end.
constexpr int kNoElem = 1 << 30;

// This lane's element offset in the row-chunk layout of a block with row stride rs, or
// kNoElem for a lane past the row (its loads then read zeros).
template <int D>
__device__ __forceinline__ int rc_lane(int l, int u, int rs) {
  return rc_valid<D>(l, u) ? rc_row<D>(l, u) * rs + rc_chunk<D>(l, u) * 8 : kNoElem;
}

// Buffer resource over one (b,h) slice of a [B,H,N,D] bf16 operand: rows [0, N) of row stride rs
// elements.  Raw buffer loads range-check each access against the slice size, so a row below 0
// (negative 32-bit offset, i.e. a huge unsigned one) or at/after N reads as zeros -- the masked
// taps cost no branch.  The caller guarantees (N + max offset) * rs * 2 < 2^31 and rs >= D, and
// N >= 1 (no kernel is launched for N = 0): the extent is then computed without a branch (one
// branch per operand split the prologue's kernel-argument loads into separately waited groups).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slice_rsrc(const bf16_t* base, long long rs,
                                                             int N, int D) {
  const int bytes = (int)(((long long)(N - 1) * rs + D) * 2);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, bytes,
                                           0x00020000);
}

// 16 bytes at element offset `elem` of a buffer (zero when out of range).
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, int elem) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)elem * 2u, 0, 0));
}

// Hides a per-lane value from the optimiser, so that (uniform row) * stride + lane_part is not
// re-associated into a per-lane (row + lane_row) * stride multiply (v_mul_lo_u32 is quarter rate).
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The long-range tap offsets as uniform values, loaded once at kernel start.  The empty asm
// fixes each value in a scalar register there; left alone, the compiler issues each kernel
// argument load at its first use inside a tap loop and waits on it (lgkmcnt(0) also waits for
// every LDS access in flight).
template <int NSM>
__device__ __forceinline__ void load_sparse_deltas(const TapTable& taps, int (&sd)[NSM]) {
#pragma unroll
  for (int t = 0; t < NSM; ++t) {
    int v = taps.sdelta[t];
    asm volatile("" : "+s"(v));
    sd[t] = v;
  }
}

// Per-lane masks that keep element e (0..3) of a 4 x bf16 operand (two dwords): the element's
// half of dword e / 2, nothing of the other dword.  A lane's e is fixed, so the masks are made
// once and each one-hot operand below costs two ANDs.
__device__ __forceinline__ uint2 onehot_masks(int e) {
  const unsigned h = (e & 1) ? 0xffff0000u : 0x0000ffffu;
  return make_uint2(e < 2 ? h : 0u, e < 2 ? 0u : h);
}

// bf16 operand that holds x in element e (masks of onehot_masks(e)) and zeros elsewhere.
__device__ __forceinline__ s16x4_t onehot_bf16x4(float x, uint2 m) {
  const unsigned p = cvt_pk_bf16(x, x);
  return __builtin_bit_cast(s16x4_t, make_uint2(p & m.x, p & m.y));
}

// Two-term bf16 split of fp32 values: x = hi + lo + O(2^-18 |x|), hi = bf16(x), lo = bf16(x - hi)
// (x - hi is exact in fp32).  An MFMA over hi and one over lo give a product with an fp32
// operand to about 2^-17 relative, where hi alone would carry 2^-9.
__device__ __forceinline__ void split_bf16x4(float a, float b, float c, float d, s16x4_t& hi,
                                             s16x4_t& lo) {
  const unsigned p0 = cvt_pk_bf16(a, b), p1 = cvt_pk_bf16(c, d);
  // The hi values back in fp32: a bf16 is the upper half of its fp32 pattern.
  const float ha = __uint_as_float(p0 << 16), hb = __uint_as_float(p0 & 0xffff0000u);
  const float hc = __uint_as_float(p1 << 16), hd = __uint_as_float(p1 & 0xffff0000u);
  hi = __builtin_bit_cast(s16x4_t, make_uint2(p0, p1));
  lo = __builtin_bit_cast(s16x4_t, make_uint2(cvt_pk_bf16(a - ha, b - hb), cvt_pk_bf16(c - hc, d - hd)));
}

// scale_embed [J, D] (fp32, 16-byte aligned) as 48 rows x DP bf16 in LDS (row stride RV; rows
// >= J and columns >= D zero), optionally with a second plane lo = bf16(se - hi).  The rows come
// in as 16-byte pieces, loaded into registers first (load) and staged later (store), so a kernel
// can issue these loads ahead of its bulk loads and wait for them alone.
template <int D>
struct SeRows {
  static constexpr int C4 = Geo<D>::DP / 4;  // 4-float pieces per staged row
  static constexpr int U = (48 * C4 + kBlock - 1) / kBlock;
  float4 x[U];
  __device__ __forceinline__ void load(const float* se, int J, int tid) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = tid + u * kBlock, j = e / C4, d = 4 * (e - j * C4);
      x[u] = se && e < 48 * C4 && j < J && d < D ? *reinterpret_cast<const float4*>(se + j * D + d)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  template <int RV>
  __device__ __forceinline__ void store(bf16_t* hi, bf16_t* lo, int tid) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = tid + u * kBlock, j = e / C4, d = 4 * (e - j * C4);
      if (e < 48 * C4) {
        s16x4_t h, o;
        split_bf16x4(x[u].x, x[u].y, x[u].z, x[u].w, h, o);
        *reinterpret_cast<uint2*>(hi + j * RV + d) = __builtin_bit_cast(uint2, h);
        if (lo) *reinterpret_cast<uint2*>(lo + j * RV + d) = __builtin_bit_cast(uint2, o);
      }
    }
  }
};

// Max / sum over the four lanes {i, i+16, i+32, i+48} that share column i of an MFMA tile.
// v_permlane16_swap / v_permlane32_swap (gfx950) hand every lane the pair {x[l], x[l^16]}
// (resp. x[l^32]) without an LDS round trip; the pair is combined in the same order on both
// lanes, so all four lanes end with bit-identical results.
__device__ __forceinline__ float xor16_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float col_max(float x) { return xor32_pair_max(xor16_pair_max(x)); }
__device__ __forceinline__ float col_sum(float x) { return xor32_pair_sum(xor16_pair_sum(x)); }

}  // namespace dsqg
