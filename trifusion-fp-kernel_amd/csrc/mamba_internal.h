// Shared declarations of the fused-recurrence kernels.
#pragma once

#include "common.h"

namespace tf {

constexpr int kChunk = 64;  // recurrence chunk length (mamba_fused.py:63)

// Valid prefix of batch row b: lengths[b] clamped to [0, T], or T.
__device__ __forceinline__ int valid_length(const tf_mamba_args& a, int b) {
  const int T = static_cast<int>(a.time);
  if (a.lengths == nullptr) return T;
  const int64_t l = a.lengths[b];
  return l < 0 ? 0 : (l > T ? T : static_cast<int>(l));
}

bool generic_supported(const tf_mamba_args& a);
int launch_generic(const tf_mamba_args& a, hipStream_t stream);

bool mfma_supported(const tf_mamba_args& a);
int launch_mfma(const tf_mamba_args& a, hipStream_t stream);
// Scratch bytes of the MFMA kernel's chunk-parallel form for these arguments
// (0: one workgroup per unit).
int64_t mfma_workspace_bytes(const tf_mamba_args& a);

// Pipelined MFMA kernel (N = P = 64): one workgroup walks each unit, or, for
// few long units with a workspace, each (unit, time segment).
bool pipe_supported(const tf_mamba_args& a);
int launch_pipe(const tf_mamba_args& a, hipStream_t stream);
// Scratch bytes of the pipelined kernel's chunk-parallel form (0: one
// workgroup per unit).
int64_t pipe_workspace_bytes(const tf_mamba_args& a);

}  // namespace tf
