// Wide-head SparseMLA kernels (d_qk = 576, d_v = 512 or 576: the DeepSeek-V3.2
// MLA latent + rope row) and the entry points the C-ABI dispatches to.
#pragma once

#include <hip/hip_runtime.h>

#include "sparse_mla_params.hpp"

namespace dsa {

// Head dims served by the wide kernels: the MLA row with its 512-dim latent as
// V, or the whole row as V (d_v defaults to d_qk when a caller passes none).
inline bool wide_shape(int64_t d_qk, int64_t d_v) { return d_qk == 576 && (d_v == 512 || d_v == 576); }

// Forward over all (token, kv group, 32-head tile) items; bf16 or e4m3.
// mx: block-scaled e4m3 kernel; qmx: bf16 kernel with Q converted from e4m3
// codes and 32-channel block scales as it is loaded
int launch_fwd_wide(const FwdParams &p, int64_t d_qk, int64_t d_v, bool fp8, hipStream_t st, bool mx = false,
                    bool qmx = false);
// Backward main pass (P, dS, dQ, fp32 partial dKV rows at CSR positions); bf16 or e4m3.
int launch_bwd_main_wide(const BwdParams &p, int64_t d_qk, int64_t d_v, bool fp8, bool f32p, hipStream_t st);

}  // namespace dsa
