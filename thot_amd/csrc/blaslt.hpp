// Plain GEMMs through hipBLASLt (see blaslt.hip).
#pragma once
#include <hip/library_types.h>
#include "nott_hip.h"

namespace nott {
namespace blas {
// Column-major D(m×n) = op(A)·op(B) + beta·D with fp32 accumulation; A and B
// of type `ab`, D of type `dt`, optional fp32 bias per row of D; `batch`
// products with element strides sa, sb, sd between them.  Returns
// NOTT_ERR_UNSUPPORTED (nothing launched) when the library has no algorithm
// for the problem, so the caller can take its own kernel.
int gemm(nott_ctx ctx, bool ta, bool tb, int64_t m, int64_t n, int64_t k, const void* A, int64_t lda, const void* B,
         int64_t ldb, hipDataType ab, void* D, int64_t ldd, hipDataType dt, float beta, const float* bias,
         int64_t batch = 1, int64_t sa = 0, int64_t sb = 0, int64_t sd = 0);
// Frees the context's handle, workspace and plans.
void release(nott_ctx ctx);
}  // namespace blas
}  // namespace nott
