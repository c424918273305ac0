// Internal: the automatic GEMM call every dl:: operation makes.
#pragma once

#include <cstdint>

namespace dl::detail {

// fdl_sgemm_ex on the current device, with a workspace from the device's
// block cache when the problem can use one (fdl_sgemm_workspace_size > 0).
// The workspace goes back to `stream`'s free list right after the enqueue:
// the next user of the block on that stream runs after this call's kernels.
// Returns the fdl status.
int sgemm_auto(int transA, int transB, int64_t M, int64_t N, int64_t K, const float* A,
               int64_t lda, int64_t strideA, const float* B, int64_t ldb, int64_t strideB,
               float* C, int64_t ldc, int64_t strideC, int64_t batch, const float* bias,
               const float* aux, int epilogue, void* stream);

}  // namespace dl::detail
