// Internal launchers shared between the kernel files and the C ABI (dsqg_abi.hip).
#pragma once

#include "dsqg_common.hpp"

namespace dsqg {

// dtype: 0 = f32, 1 = bf16.  Each returns hipGetLastError() after its launches, or
// hipErrorInvalidValue for a head dim without a kernel (the ABI checks that first).
hipError_t launch_fwd(const FwdParams& p, int dtype, int D, hipStream_t st);

// bf16 MFMA forward (dsqg_fwd_mfma.hip): head dims 32/64/128, at most kMaxSparse taps beyond
// the dense window, row strides >= D and 32-bit byte offsets within each (b,h) slice.
// launch_fwd picks it whenever it applies.
bool fwd_mfma_supported(const FwdParams& p, int D);
hipError_t launch_fwd_mfma(const FwdParams& p, int D, hipStream_t st);

// Tiling of the backward for these sizes and kernel choice; fills n_tiles / tiles_per_block /
// n_chunks / n_tiles_kv (se: scale_embed or its gradient is present).
void bwd_plan(BwdParams& p, int D, int dtype, bool se);

// bf16 MFMA backward kernels: same conditions as the MFMA forward.
bool bwd_mfma_supported(const BwdParams& p, int D, int dtype);
hipError_t launch_bwd_dq_mfma(const BwdParams& p, int D, unsigned nblocks, hipStream_t st);
hipError_t launch_bwd_dkdv_mfma(const BwdParams& p, int D, unsigned nblocks, hipStream_t st);
hipError_t launch_bwd_reduce(const ReduceParams& r, hipStream_t st);
// dscale_embed's first reduction stage alone (a no-op without dscale_embed), and the rest.
hipError_t launch_bwd_reduce_se_stage(const ReduceParams& r, hipStream_t st);
hipError_t launch_bwd_reduce_final(const ReduceParams& r, hipStream_t st);
// dk/dv and then the parameter reduction r: with the bf16 MFMA dk/dv kernel the reduction
// rides in the same launch as extra workgroups; otherwise two launches.  r's dscale_embed
// first stage must already have run.
hipError_t launch_bwd_dkdv_params(const BwdParams& p, const ReduceParams& r, int dtype, int D,
                                  unsigned nblocks, hipStream_t st);
hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int D, unsigned nblocks, hipStream_t st);
hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int D, unsigned nblocks, hipStream_t st);

hipError_t launch_decode(const DecodeParams& p, int dtype, int D, hipStream_t st);

bool head_dim_supported(int D);

}  // namespace dsqg
