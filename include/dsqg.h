/*
 * dsqg.h -- C ABI of libdsqg_hip.so, the MI355X (gfx950) DSQG fixed-offset sparse attention.
 *
 * DSQG attention: query row n of head (b,h) attends the J keys n - delta_j of the same head,
 * for a fixed, sorted offset table delta_0 < delta_1 < ... < delta_{J-1}.  With c = 1/sqrt(D):
 *
 *     s_j   = g[h,j] * c * q_n . k_{n-delta_j} + pos_bias[j,h] + c * q_n . se_j
 *     alpha = softmax_j(s) over the valid taps (n - delta_j >= 0); invalid taps have weight 0,
 *             are excluded from the normalisation and are never dereferenced
 *     out_n = a[h] * sum_j alpha_j v_{n-delta_j},     lse_n = logsumexp_j(s_j)
 *
 * g (score_gain, [H,J]) and a (if_gain, [H]) are optional (NULL means 1); se (scale_embed,
 * [J,D]) is optional (NULL means 0).  pos_bias is [J,H], as in the reference.
 *
 * Conventions.
 *  - Every entry point returns a dsqg_status.  Argument checks happen on the host before any
 *    HIP call, so a bad call never launches a kernel.
 *  - The library never allocates device memory and never synchronises; all work is ordered on
 *    the stream passed in.  Its only mutable global state is dsqg_bwd_noalloc's per-device
 *    static scratch (below); every other entry point is re-entrant.
 *  - Tensor pointers are device pointers.  Element strides are int64 element counts, in the
 *    order [B,H,N,D]; the innermost (D) stride must be 1 and the other strides and the base
 *    pointers must keep every row 16-byte aligned.
 *  - pos_bias / scale_embed / score_gain / if_gain and the parameter gradients are fp32 and
 *    contiguous; dsqg_fwd and dsqg_bwd also need scale_embed (when given) 16-byte aligned.  q/k/v/out/dout/dq/dk/dv share one element type (dtype).
 *
 * Reference interfaces replaced (paths are in the Lanerra/DWARF tree):
 *  - dsqg_fwd        <- _DSQGFnV3.forward, kernels/dsqg_attention_v3.py:361-387
 *                       (and the pybind forward(q,k,v,pb,se) of
 *                        kernels/dsqg_cuda/dsqg_cuda_kernel.cu:496-530)
 *  - dsqg_bwd        <- _DSQGFnV3.backward, kernels/dsqg_attention_v3.py:389-442
 *                       (pybind backward(...) of kernels/dsqg_cuda/dsqg_cuda_kernel.cu:532-609)
 *  - dsqg_decode_step: no counterpart in the reference, which regenerates the whole prefix for
 *                       every token (train/train_2048_condU.py:463-487); it realises the
 *                       circular K/V buffer described in README.md:175-177.
 *  - dsqg_pool_gate_fwd / _bwd <- the interference pool of DSQGBlock.forward,
 *                       train/train_2048_condU.py:289-292 (cumsum / counts, sigmoid gate), and
 *                       its autograd backward.
 */
#ifndef DWARF_DSQG_H
#define DWARF_DSQG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSQG_ABI_VERSION 3
#define DSQG_MAX_OFFSETS 64

/* Same type as hipStream_t; NULL is the null stream. */
typedef struct ihipStream_t* dsqg_stream_t;

typedef enum {
    DSQG_OK = 0,
    DSQG_EINVAL = 1,        /* bad shape, stride, alignment, pointer or offset table */
    DSQG_EUNSUPPORTED = 2,  /* valid arguments this build has no kernel for: the head dim,
                               J > 48, or (bf16) more than 16 offsets beyond the dense
                               window delta = 0, 1, 2, ... or a slice whose rows a 32-bit
                               byte offset cannot reach */
    DSQG_EHIP = 3,          /* a HIP launch failed (hipGetLastError after the launch) */
    DSQG_EWORKSPACE = 4,    /* workspace pointer NULL or smaller than required */
    DSQG_ETOOLARGE = 5      /* dsqg_bwd_noalloc: the call needs more than its static scratch */
} dsqg_status;

/* Static scratch of dsqg_bwd_noalloc (bytes per device): the backward workspace of the largest
 * call it takes, as dsqg_bwd_workspace_size reports it (e.g. 37 MB for B8 H12 N2048 D64 with
 * dscale_embed, 1.3 MB without). */
#define DSQG_NOALLOC_SCRATCH_BYTES (64u << 20)

/* DSQG_F16 is accepted by the pool entry points only. */
typedef enum { DSQG_F32 = 0, DSQG_BF16 = 1, DSQG_F16 = 2 } dsqg_dtype;

/* Shape and offset table shared by all entry points. */
typedef struct {
    int32_t dtype;                       /* dsqg_dtype */
    int32_t B, H, N, D;                  /* N is ignored by the decode step */
    int32_t J;                           /* number of offsets, 1..DSQG_MAX_OFFSETS; this
                                            build's kernels take J <= 48 (else EUNSUPPORTED) */
    int32_t offsets[DSQG_MAX_OFFSETS];   /* strictly increasing, offsets[0] == 0 */
} dsqg_shape;

/* Forward: out [B,H,N,D] (dtype), lse [B,H,N] fp32 contiguous (lse may be NULL).
 * alpha_lr (bf16 only; NULL = not written, and ignored for fp32): the softmax weights of the
 * long-range taps, [B,H,NS,N] fp32 contiguous with NS = dsqg_long_range_taps(offsets): saved
 * for the bf16 backward, which requires them (as the reference saves out and lse,
 * kernels/dsqg_attention_v3.py:384); dsqg_alpha_lr_elems gives its size.
 * Replaces kernels/dsqg_attention_v3.py:361-387 (_DSQGFnV3.forward). */
typedef struct {
    dsqg_shape shape;
    const void* q;  int64_t q_stride[4];
    const void* k;  int64_t k_stride[4];
    const void* v;  int64_t v_stride[4];
    const float* pos_bias;     /* [J,H] */
    const float* scale_embed;  /* [J,D] or NULL */
    const float* score_gain;   /* [H,J] or NULL */
    const float* if_gain;      /* [H]   or NULL */
    void* out;  int64_t out_stride[4];
    float* lse;                /* [B,H,N] or NULL */
    float* alpha_lr;           /* [B,H,NS,N] or NULL (bf16) */
} dsqg_fwd_args;

/* Backward.  dout is the gradient of out; lse and (bf16, required when the table has taps
 * beyond its dense window) alpha_lr are the forward's.  dq/dk/dv are written
 * (not accumulated).  dpos_bias [J,H] is required; dscale_embed [J,D], dscore_gain [H,J] and
 * dif_gain [H] are written when non-NULL (they are defined even when the matching input is
 * NULL, i.e. at se = 0, g = 1, a = 1).  The parameter gradients are reduced
 * deterministically from per-workgroup partials in the workspace (no global atomics).
 * Replaces kernels/dsqg_attention_v3.py:389-442 (_DSQGFnV3.backward). */
typedef struct {
    dsqg_shape shape;
    const void* q;    int64_t q_stride[4];
    const void* k;    int64_t k_stride[4];
    const void* v;    int64_t v_stride[4];
    const void* dout; int64_t dout_stride[4];
    const float* lse;          /* [B,H,N] */
    const float* pos_bias;     /* [J,H] */
    const float* scale_embed;  /* [J,D] or NULL */
    const float* score_gain;   /* [H,J] or NULL */
    const float* if_gain;      /* [H]   or NULL */
    void* dq;  int64_t dq_stride[4];
    void* dk;  int64_t dk_stride[4];
    void* dv;  int64_t dv_stride[4];
    float* dpos_bias;          /* [J,H] */
    float* dscale_embed;       /* [J,D] or NULL */
    float* dscore_gain;        /* [H,J] or NULL */
    float* dif_gain;           /* [H]   or NULL */
    void* workspace;           /* device memory, 256-byte aligned */
    size_t workspace_bytes;
    const float* alpha_lr;     /* [B,H,NS,N] from dsqg_fwd (bf16); ignored for fp32 */
} dsqg_bwd_args;

/* Decode step: one new token per sequence.  q, k_new, v_new, out are [B,H,D] contiguous;
 * k_ring, v_ring are [B,H,S,D] contiguous rings with S > max(offsets) and S*D*sizeof(dtype) < 2^31
 * (DSQG_EUNSUPPORTED otherwise).  pos [B] (device,
 * int64) is the absolute position of the new token.  The step writes k_new / v_new into slot
 * pos mod S, then attends slot (pos - delta_j) mod S for delta_j > 0 and the new row for
 * delta_j == 0; taps with pos - delta_j < 0 are masked (never wrapped).  If pos_next is non-NULL
 * (and distinct from pos) it receives pos + 1, so a captured step can be replayed.  A negative
 * pos marks an invalid sequence: its output is NaN, its rings are untouched, and pos_next
 * receives the same negative value, so it stays invalid over replays. */
typedef struct {
    dsqg_shape shape;
    int32_t S;                 /* ring slots */
    const void* q;
    const void* k_new;
    const void* v_new;
    void* k_ring;
    void* v_ring;
    const int64_t* pos;        /* [B] */
    int64_t* pos_next;         /* [B] or NULL */
    const float* pos_bias;     /* [J,H] */
    const float* scale_embed;  /* [J,D] or NULL */
    const float* score_gain;   /* [H,J] or NULL */
    const float* if_gain;      /* [H]   or NULL */
    void* out;
} dsqg_decode_args;

int dsqg_abi_version(void);
const char* dsqg_status_string(int status);

/* Head dims this build has kernels for, written to dims (up to cap entries); returns the
 * count. */
int dsqg_supported_head_dims(int32_t* dims, int cap);

int dsqg_fwd(const dsqg_fwd_args* args, dsqg_stream_t stream);

/* Taps beyond the dense window of an offset table (offsets[0..W] = 0..W, W <= 32): the NS of
 * alpha_lr.  Returns NS >= 0, or a negative DSQG_EINVAL for an invalid table. */
int dsqg_long_range_taps(const int32_t* offsets, int J);

/* Elements of alpha_lr for a shape (B * H * NS * N; 0 for fp32).  Returns DSQG_OK and writes
 * *elems, or an argument error.  No counterpart in the reference (which recomputes every score
 * in its backward). */
int dsqg_alpha_lr_elems(const dsqg_shape* shape, size_t* elems);

/* Workspace the backward needs for these arguments (shape and which gradients are requested).
 * Returns DSQG_OK and writes *bytes, or an argument error. */
int dsqg_bwd_workspace_size(const dsqg_bwd_args* args, size_t* bytes);
int dsqg_bwd(const dsqg_bwd_args* args, dsqg_stream_t stream);

/* The three phases dsqg_bwd runs, for callers that launch them separately (the reference's
 * backward is likewise three launches: kernels/dsqg_attention_v3.py:397-441).  Call them in
 * this order on one stream with the same args and workspace: the workspace carries D', (bf16)
 * the long-range taps' dk/dv weights and the parameter-gradient partials from phase 1 to
 * phases 2 and 3.
 *  - dsqg_bwd_dq     <- _compute_D_v3 + _bwd_dq_v3 (:397-424): dq, D', partials, and for bf16
 *                       the weights (c g dS, a alpha) of every query's long-range taps
 *  - dsqg_bwd_dkdv   <- _bwd_dkdv_v3 (:426-441): dk, dv
 *  - dsqg_bwd_params <- the tl.atomic_add accumulation of dpb/dse in _bwd_dq_v3 (:265-271),
 *                       here a deterministic reduction of the partials */
int dsqg_bwd_dq(const dsqg_bwd_args* args, dsqg_stream_t stream);
int dsqg_bwd_dkdv(const dsqg_bwd_args* args, dsqg_stream_t stream);
int dsqg_bwd_params(const dsqg_bwd_args* args, dsqg_stream_t stream);

/* dsqg_bwd without a workspace argument and without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  args->workspace and workspace_bytes
 * are ignored; the workspace is a static scratch array of DSQG_NOALLOC_SCRATCH_BYTES on each
 * device.  That array is part of the library's code object, so it takes its 64 MiB of device
 * memory on every device where the library is loaded, whether or not this entry point is ever
 * called.  Its address is looked up once per device on the first call there (hipGetSymbolAddress):
 * make that first call outside stream capture (one eager call), later calls may be captured
 * into a HIP graph (the call issues kernel launches only, no memset and no allocation).  A call whose
 * workspace (dsqg_bwd_workspace_size) exceeds it returns DSQG_ETOOLARGE before any HIP call.
 * Same kernels, outputs and stream rules as dsqg_bwd; calls that overlap on one device (other
 * streams, other threads) share the scratch and race, so serialise them. */
int dsqg_bwd_noalloc(const dsqg_bwd_args* args, dsqg_stream_t stream);

int dsqg_decode_step(const dsqg_decode_args* args, dsqg_stream_t stream);

/* Causal-mean pool with a sigmoid gate (the interference branch of a DWARF block):
 *
 *     pool[b,n,c] = (sum_{m<=n} x[b,m,c]) / (n + 1)
 *     out[b,n,c]  = s[b,n,c] * pool[b,n,c],         s = sigmoid(gate_pre), rounded to gate_dtype
 *
 * x, gate_pre and out are [B,N,C] with element strides {b, n} and unit channel stride; C must
 * be a multiple of 8, base pointers and rows 16-byte aligned, the row stride at least C (rows do
 * not overlap) and one batch slice under 2 GiB (EUNSUPPORTED otherwise).  Each tensor has its own element
 * type (F32, BF16 or F16); arithmetic is fp32 and the sums are deterministic.  The workspace
 * (size from dsqg_pool_gate_workspace_size, 256-byte aligned) holds per-chunk column sums.
 * Replaces train/train_2048_condU.py:289-292 (pool = xi.cumsum(1) / counts;
 * inter = sigmoid(inter_gate(xi)) * pool). */
typedef struct {
    int32_t B, N, C;
    int32_t x_dtype, gate_dtype, out_dtype;   /* dsqg_dtype each */
    const void* x;         int64_t x_stride[2];
    const void* gate_pre;  int64_t gate_stride[2];
    void* out;             int64_t out_stride[2];
    void* workspace;
    size_t workspace_bytes;
} dsqg_pool_gate_fwd_args;

/* Backward of dsqg_pool_gate_fwd for dout = d out (element type out_dtype):
 *
 *     dgate_pre[b,n,c] = dout * pool * s * (1 - s)                 (gate_dtype)
 *     dx[b,m,c]        = sum_{n>=m} dout[b,n,c] * s[b,n,c] / (n+1)  (x_dtype)
 *
 * Either output may be NULL (not computed).  Layout rules as for the forward.
 * Replaces torch autograd through train/train_2048_condU.py:289-292. */
typedef struct {
    int32_t B, N, C;
    int32_t x_dtype, gate_dtype, dout_dtype;  /* dsqg_dtype each */
    const void* x;         int64_t x_stride[2];
    const void* gate_pre;  int64_t gate_stride[2];
    const void* dout;      int64_t dout_stride[2];
    void* dx;              int64_t dx_stride[2];
    void* dgate_pre;       int64_t dgate_stride[2];
    void* workspace;
    size_t workspace_bytes;
} dsqg_pool_gate_bwd_args;

/* Workspace bytes of dsqg_pool_gate_fwd (backward == 0) or _bwd (backward != 0). */
int dsqg_pool_gate_workspace_size(int32_t B, int32_t N, int32_t C, int backward, size_t* bytes);
int dsqg_pool_gate_fwd(const dsqg_pool_gate_fwd_args* args, dsqg_stream_t stream);
int dsqg_pool_gate_bwd(const dsqg_pool_gate_bwd_args* args, dsqg_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DWARF_DSQG_H */
