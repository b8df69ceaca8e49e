// C ABI of libdsqg_hip.so (declared in include/dsqg.h).  Every entry point validates its
// arguments on the host before touching HIP, then fills a launch parameter block and
// dispatches on (dtype, head dim, offset count).  No allocation and no synchronisation; the
// only mutable global state is dsqg_bwd_noalloc's per-device static scratch (end of file).
#include <limits.h>
#include <math.h>
#include <string.h>

#include <mutex>

#include "../../include/dsqg.h"
#include "dsqg_common.hpp"
#include "dsqg_launch.hpp"

using namespace dsqg;

namespace {

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

size_t elem_size(int dtype) { return dtype == DSQG_F32 ? 4 : 2; }

// Validates the shape block and derives the tap table (dense window W, max offset).
int check_shape(const dsqg_shape& s, bool need_n, TapTable* taps) {
  if (s.dtype != DSQG_F32 && s.dtype != DSQG_BF16) return DSQG_EINVAL;
  if (s.B < 0 || s.H < 0 || s.D <= 0 || (need_n && s.N < 0)) return DSQG_EINVAL;
  if (s.J < 1 || s.J > DSQG_MAX_OFFSETS) return DSQG_EINVAL;
  if (s.offsets[0] != 0) return DSQG_EINVAL;
  for (int j = 1; j < s.J; ++j)
    if (s.offsets[j] <= s.offsets[j - 1] || s.offsets[j] > (1 << 28)) return DSQG_EINVAL;
  if (!head_dim_supported(s.D) || s.J > kMaxTaps) return DSQG_EUNSUPPORTED;
  taps->J = s.J;
  taps->maxd = s.offsets[s.J - 1];
  int W = 0;
  while (W + 1 < s.J && W + 1 <= kMaxWindow && s.offsets[W + 1] == W + 1) ++W;
  taps->W = W;
  for (int j = 0; j < kMaxOffsets; ++j) taps->delta[j] = j < s.J ? s.offsets[j] : 0;
  for (int t = 0; t < kMaxSparse; ++t) taps->sdelta[t] = W + 1 + t < s.J ? s.offsets[W + 1 + t] : 0;
  return DSQG_OK;
}

// A [B,H,N,D] operand: non-null when non-empty, 16-byte aligned rows, unit D stride,
// non-negative strides.
int check_tensor(const void* ptr, const int64_t st[4], int dtype, long long nelem) {
  if (nelem == 0) return DSQG_OK;
  if (!ptr || !aligned16(ptr)) return DSQG_EINVAL;
  if (st[3] != 1) return DSQG_EINVAL;
  const size_t es = elem_size(dtype);
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || (st[i] * (int64_t)es) % 16 != 0) return DSQG_EINVAL;
  return DSQG_OK;
}

Strides4 to_strides(const int64_t st[4]) { return Strides4{st[0], st[1], st[2], st[3]}; }

int hip_status(hipError_t e) { return e == hipSuccess ? DSQG_OK : DSQG_EHIP; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct BwdLayout {
  size_t dpre, lrw, part_bias, part_gain, part_if, part_se, se_stage, total;
  int se_slices, se_per;  // two-stage dscale_embed sum: slices of se_per workgroup partials
};

constexpr size_t kMaxSeSlices = 256;

BwdLayout bwd_layout(const dsqg_bwd_args& a, const BwdParams& p) {
  const dsqg_shape& s = a.shape;
  const size_t nb = (size_t)p.n_bgroups * s.H * p.n_chunks;
  BwdLayout L{};
  size_t off = 0;
  L.dpre = off; off = align256(off + sizeof(float) * (size_t)s.B * s.H * s.N);
  // bf16: the long-range taps' dk/dv weights, a bf16 pair per (b, h, tap, row), from dq to dk/dv.
  L.lrw = off;
  if (s.dtype == DSQG_BF16)
    off = align256(off + sizeof(unsigned) * (size_t)s.B * s.H * s.N * (p.taps.J - p.taps.W - 1));
  L.part_bias = off; off = align256(off + sizeof(float) * nb * s.J);
  L.part_gain = off; if (a.dscore_gain) off = align256(off + sizeof(float) * nb * s.J);
  L.part_if = off; if (a.dif_gain) off = align256(off + sizeof(float) * nb);
  L.part_se = off; if (a.dscale_embed) off = align256(off + sizeof(float) * nb * s.J * s.D);
  L.se_slices = 0; L.se_per = 0;
  if (nb > 0) {
    L.se_per = (int)((nb + kMaxSeSlices - 1) / kMaxSeSlices);
    L.se_slices = (int)((nb + L.se_per - 1) / L.se_per);
  }
  L.se_stage = off; if (a.dscale_embed) off = align256(off + sizeof(float) * L.se_slices * s.J * s.D);
  L.total = off;
  return L;
}

int check_bwd(const dsqg_bwd_args* a, BwdParams* p) {
  if (!a) return DSQG_EINVAL;
  const dsqg_shape& s = a->shape;
  memset(p, 0, sizeof(*p));
  int st = check_shape(s, true, &p->taps);
  if (st) return st;
  const long long ne = (long long)s.B * s.H * s.N * s.D;
  if ((st = check_tensor(a->q, a->q_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->k, a->k_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->v, a->v_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->dout, a->dout_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->dq, a->dq_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->dk, a->dk_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->dv, a->dv_stride, s.dtype, ne))) return st;
  if (ne > 0 && !a->lse) return DSQG_EINVAL;
  // bf16: the forward's long-range weights (4-byte aligned fp32) whenever there are such taps.
  if (s.dtype == DSQG_BF16 && ne > 0 && p->taps.J - p->taps.W - 1 > 0 &&
      (!a->alpha_lr || (reinterpret_cast<uintptr_t>(a->alpha_lr) & 3u) != 0))
    return DSQG_EINVAL;
  if ((long long)s.J * s.H > 0 && (!a->pos_bias || !a->dpos_bias)) return DSQG_EINVAL;
  if (!aligned16(a->scale_embed)) return DSQG_EINVAL;  // read as 16-byte pieces
  p->B = s.B; p->H = s.H; p->N = s.N;
  p->qs = to_strides(a->q_stride); p->ks = to_strides(a->k_stride);
  p->vs = to_strides(a->v_stride); p->dos = to_strides(a->dout_stride);
  bwd_plan(*p, s.D, s.dtype, a->scale_embed != nullptr || a->dscale_embed != nullptr);
  if (s.dtype == DSQG_BF16 && !bwd_mfma_supported(*p, s.D, s.dtype)) return DSQG_EUNSUPPORTED;
  if ((long long)s.B * s.H * p->n_chunks > INT_MAX / 2) return DSQG_EINVAL;  // >= the partial count
  if ((long long)s.B * s.H * p->n_tiles_kv > INT_MAX / 2) return DSQG_EINVAL;
  return DSQG_OK;
}

}  // namespace

extern "C" {

int dsqg_abi_version(void) { return DSQG_ABI_VERSION; }

const char* dsqg_status_string(int status) {
  switch (status) {
    case DSQG_OK: return "ok";
    case DSQG_EINVAL: return "invalid argument (shape, stride, alignment, pointer or offset table)";
    case DSQG_EUNSUPPORTED:
      return "unsupported configuration (head dim, more than 48 offsets, or a bf16 table with "
             "more than 16 offsets beyond the dense window)";
    case DSQG_EHIP: return "HIP launch error";
    case DSQG_EWORKSPACE: return "workspace missing or too small";
    case DSQG_ETOOLARGE:
      return "the call needs more workspace than dsqg_bwd_noalloc's static scratch "
             "(DSQG_NOALLOC_SCRATCH_BYTES); use dsqg_bwd with a workspace";
    default: return "unknown status";
  }
}

int dsqg_supported_head_dims(int32_t* dims, int cap) {
  static const int32_t kDims[] = {32, 64, 80, 96, 128};
  const int n = (int)(sizeof(kDims) / sizeof(kDims[0]));
  for (int i = 0; i < n && i < cap; ++i) dims[i] = kDims[i];
  return n;
}

int dsqg_fwd(const dsqg_fwd_args* a, dsqg_stream_t stream) {
  if (!a) return DSQG_EINVAL;
  const dsqg_shape& s = a->shape;
  FwdParams p;
  memset(&p, 0, sizeof(p));
  int st = check_shape(s, true, &p.taps);
  if (st) return st;
  const long long ne = (long long)s.B * s.H * s.N * s.D;
  if ((st = check_tensor(a->q, a->q_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->k, a->k_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->v, a->v_stride, s.dtype, ne))) return st;
  if ((st = check_tensor(a->out, a->out_stride, s.dtype, ne))) return st;
  if ((long long)s.J * s.H > 0 && !a->pos_bias) return DSQG_EINVAL;
  if (!aligned16(a->scale_embed)) return DSQG_EINVAL;  // read as 16-byte pieces
  if ((long long)s.B * s.H * ((s.N + 15) / 16) > INT_MAX / 2) return DSQG_EINVAL;
  if (ne == 0) return DSQG_OK;
  p.B = s.B; p.H = s.H; p.N = s.N;
  p.scale = 1.0f / sqrtf((float)s.D);
  p.q = a->q; p.qs = to_strides(a->q_stride);
  p.k = a->k; p.ks = to_strides(a->k_stride);
  p.v = a->v; p.vs = to_strides(a->v_stride);
  p.pos_bias = a->pos_bias; p.scale_embed = a->scale_embed;
  p.score_gain = a->score_gain; p.if_gain = a->if_gain;
  p.out = a->out; p.os = to_strides(a->out_stride);
  p.lse = a->lse;
  p.alpha_lr = s.dtype == DSQG_BF16 ? a->alpha_lr : nullptr;
  // bf16 has one implementation, the MFMA kernel: tables with more long-range taps than it
  // holds, or slices beyond its 32-bit offsets, are not taken.
  if (s.dtype == DSQG_BF16 && !fwd_mfma_supported(p, s.D)) return DSQG_EUNSUPPORTED;
  return hip_status(launch_fwd(p, s.dtype, s.D, reinterpret_cast<hipStream_t>(stream)));
}

int dsqg_long_range_taps(const int32_t* offsets, int J) {
  if (!offsets) return -DSQG_EINVAL;
  dsqg_shape s;
  memset(&s, 0, sizeof(s));
  s.dtype = DSQG_BF16; s.D = 64; s.J = J;
  if (J < 1 || J > DSQG_MAX_OFFSETS) return -DSQG_EINVAL;
  for (int j = 0; j < J; ++j) s.offsets[j] = offsets[j];
  TapTable taps;
  const int st = check_shape(s, true, &taps);
  if (st == DSQG_EINVAL) return -DSQG_EINVAL;
  int W = 0;
  while (W + 1 < J && W + 1 <= kMaxWindow && offsets[W + 1] == W + 1) ++W;
  return J - W - 1;
}

int dsqg_alpha_lr_elems(const dsqg_shape* shape, size_t* elems) {
  if (!shape || !elems) return DSQG_EINVAL;
  TapTable taps;
  const int st = check_shape(*shape, true, &taps);
  if (st) return st;
  *elems = shape->dtype == DSQG_BF16
               ? (size_t)shape->B * shape->H * shape->N * (size_t)(taps.J - taps.W - 1) : 0;
  return DSQG_OK;
}

int dsqg_bwd_workspace_size(const dsqg_bwd_args* a, size_t* bytes) {
  if (!bytes) return DSQG_EINVAL;
  BwdParams p;
  int st = check_bwd(a, &p);
  if (st) return st;
  *bytes = bwd_layout(*a, p).total;
  return DSQG_OK;
}

// Phase selector for the backward entry points.
enum { kPhaseDq = 1, kPhaseDkdv = 2, kPhaseParams = 4, kPhaseAll = 7 };

// Workspace source of a backward call: the caller's (args->workspace), or the static scratch
// of dsqg_bwd_noalloc.
static int scratch_for_stream(hipStream_t st, void** ptr);

static int run_bwd(const dsqg_bwd_args* a, int phases, dsqg_stream_t stream, bool use_scratch) {
  BwdParams p;
  int st = check_bwd(a, &p);
  if (st) return st;
  const dsqg_shape& s = a->shape;
  const BwdLayout L = bwd_layout(*a, p);
  char* ws = static_cast<char*>(a->workspace);
  if (use_scratch) {
    // Sizes are checked before any HIP call; the scratch pointer of this stream's device is
    // taken (once per device) only for a call that fits.
    if (L.total > DSQG_NOALLOC_SCRATCH_BYTES) return DSQG_ETOOLARGE;
    void* sp = nullptr;
    if (L.total > 0 && (st = scratch_for_stream(reinterpret_cast<hipStream_t>(stream), &sp))) return st;
    ws = static_cast<char*>(sp);
  } else if (L.total > 0) {
    if (!a->workspace || a->workspace_bytes < L.total) return DSQG_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0) return DSQG_EINVAL;
  }
  p.scale = 1.0f / sqrtf((float)s.D);
  p.q = a->q; p.qs = to_strides(a->q_stride);
  p.k = a->k; p.ks = to_strides(a->k_stride);
  p.v = a->v; p.vs = to_strides(a->v_stride);
  p.dout = a->dout; p.dos = to_strides(a->dout_stride);
  p.lse = a->lse;
  p.alpha_lr = a->alpha_lr;
  p.pos_bias = a->pos_bias; p.scale_embed = a->scale_embed;
  p.score_gain = a->score_gain; p.if_gain = a->if_gain;
  p.dq = a->dq; p.dqs = to_strides(a->dq_stride);
  p.dk = a->dk; p.dks = to_strides(a->dk_stride);
  p.dv = a->dv; p.dvs = to_strides(a->dv_stride);
  p.dpre = reinterpret_cast<float*>(ws + L.dpre);
  p.lrw = reinterpret_cast<float*>(ws + L.lrw);
  p.part_bias = reinterpret_cast<float*>(ws + L.part_bias);
  p.part_gain = a->dscore_gain ? reinterpret_cast<float*>(ws + L.part_gain) : nullptr;
  p.part_if = a->dif_gain ? reinterpret_cast<float*>(ws + L.part_if) : nullptr;
  p.part_se = a->dscale_embed ? reinterpret_cast<float*>(ws + L.part_se) : nullptr;

  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  const bool rows = (long long)s.B * s.H * s.N > 0;
  ReduceParams r;
  memset(&r, 0, sizeof(r));
  r.B = p.n_bgroups; r.H = s.H; r.J = s.J; r.D = s.D;
  r.n_chunks = rows ? p.n_chunks : 0;  // no rows: the empty sums write zeros
  r.part_bias = p.part_bias; r.part_se = p.part_se;
  r.part_gain = p.part_gain; r.part_if = p.part_if;
  r.dpos_bias = a->dpos_bias; r.dscale_embed = a->dscale_embed;
  r.dscore_gain = a->dscore_gain; r.dif_gain = a->dif_gain;
  r.se_stage = a->dscale_embed ? reinterpret_cast<float*>(ws + L.se_stage) : nullptr;
  r.se_slices = rows ? L.se_slices : 0;
  r.se_per = L.se_per;
  const unsigned nb_dq = (unsigned)((long long)p.n_bgroups * s.H * p.n_chunks);
  const unsigned nb_kv = (unsigned)((long long)s.B * s.H * p.n_tiles_kv);
  if (phases == kPhaseAll && rows) {
    // dq (with the partials), dscale_embed's first stage, then dk/dv with the rest of the
    // parameter reduction in the same launch.
    if ((st = hip_status(launch_bwd_dq(p, s.dtype, s.D, nb_dq, hs)))) return st;
    if ((st = hip_status(launch_bwd_reduce_se_stage(r, hs)))) return st;
    return hip_status(launch_bwd_dkdv_params(p, r, s.dtype, s.D, nb_kv, hs));
  }
  if ((phases & kPhaseDq) && rows) {
    if ((st = hip_status(launch_bwd_dq(p, s.dtype, s.D, nb_dq, hs)))) return st;
  }
  if ((phases & kPhaseDkdv) && rows) {
    if ((st = hip_status(launch_bwd_dkdv(p, s.dtype, s.D, nb_kv, hs)))) return st;
  }
  if (phases & kPhaseParams) {
    if ((st = hip_status(launch_bwd_reduce(r, hs)))) return st;
  }
  return DSQG_OK;
}

int dsqg_bwd(const dsqg_bwd_args* a, dsqg_stream_t stream) {
  return run_bwd(a, kPhaseAll, stream, false);
}
int dsqg_bwd_dq(const dsqg_bwd_args* a, dsqg_stream_t stream) {
  return run_bwd(a, kPhaseDq, stream, false);
}
int dsqg_bwd_dkdv(const dsqg_bwd_args* a, dsqg_stream_t stream) {
  return run_bwd(a, kPhaseDkdv, stream, false);
}
int dsqg_bwd_params(const dsqg_bwd_args* a, dsqg_stream_t stream) {
  return run_bwd(a, kPhaseParams, stream, false);
}
int dsqg_bwd_noalloc(const dsqg_bwd_args* a, dsqg_stream_t stream) {
  return run_bwd(a, kPhaseAll, stream, true);
}

int dsqg_decode_step(const dsqg_decode_args* a, dsqg_stream_t stream) {
  if (!a) return DSQG_EINVAL;
  const dsqg_shape& s = a->shape;
  DecodeParams p;
  memset(&p, 0, sizeof(p));
  int st = check_shape(s, false, &p.taps);
  if (st) return st;
  if (a->S <= p.taps.maxd) return DSQG_EINVAL;
  const long long ring_bytes = (long long)a->S * s.D * (s.dtype == DSQG_F32 ? 4 : 2);
  if (ring_bytes >= (1LL << 31)) return DSQG_EUNSUPPORTED;  // ring byte offsets are 32-bit
  const long long rows = (long long)s.B * s.H;
  if (rows == 0) return DSQG_OK;
  const void* ptrs[] = {a->q, a->k_new, a->v_new, a->k_ring, a->v_ring, a->out};
  for (const void* ptr : ptrs)
    if (!ptr || !aligned16(ptr)) return DSQG_EINVAL;
  if (!a->pos || !a->pos_bias) return DSQG_EINVAL;
  if (a->pos_next && a->pos_next == a->pos) return DSQG_EINVAL;
  if (rows > INT_MAX) return DSQG_EINVAL;
  if (s.H > 4 * 65535) return DSQG_EUNSUPPORTED;  // grid: B sequences x ceil(H / 4) head groups
  p.B = s.B; p.H = s.H; p.S = a->S;
  p.scale = 1.0f / sqrtf((float)s.D);
  p.q = a->q; p.k_new = a->k_new; p.v_new = a->v_new;
  p.k_ring = a->k_ring; p.v_ring = a->v_ring;
  p.pos = reinterpret_cast<const long long*>(a->pos);
  p.pos_next = reinterpret_cast<long long*>(a->pos_next);
  p.pos_bias = a->pos_bias; p.scale_embed = a->scale_embed;
  p.score_gain = a->score_gain; p.if_gain = a->if_gain;
  p.out = a->out;
  return hip_status(launch_decode(p, s.dtype, s.D, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"

namespace dsqg {
bool head_dim_supported(int D) { return D == 32 || D == 64 || D == 80 || D == 96 || D == 128; }
}  // namespace dsqg

// ---------------------------------------------------------------------------------------------
// Static scratch of dsqg_bwd_noalloc: the backward's workspace (D', parameter-gradient partials)
// in a file-scope device array, so that the call allocates nothing.  Each device the library
// runs on holds its own copy for the life of the process.  Host code never uses the array's
// name as an address (on the host it is only a stand-in): the device address comes from
// hipGetSymbolAddress, taken once per device with that device current, and is kept per device.
// Every word the kernels read is written earlier in the same call, so nothing needs clearing
// between calls; calls that overlap on one device share the array and race.
// ---------------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[DSQG_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

static int scratch_for_stream(hipStream_t st, void** ptr) {
  int dev = -1;
  if (st) {
    if (hipStreamGetDevice(st, &dev) != hipSuccess) return DSQG_EHIP;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return DSQG_EHIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return DSQG_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return DSQG_EHIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return DSQG_EHIP;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return DSQG_EHIP;
    if (e != hipSuccess || !p) return DSQG_EHIP;
    if ((reinterpret_cast<uintptr_t>(p) & 255u) != 0) return DSQG_EHIP;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return DSQG_OK;
}
