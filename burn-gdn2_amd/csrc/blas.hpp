// Row-major f32 GEMMs of the layer: C[M, N] = op(A) op(B) (+ beta C) through
// hipBLASLt, with one plan (descriptors + algorithm) cached per shape.  The
// algorithm is the fastest of the heuristic's first 32 candidates, timed on
// the first call's operands into a scratch output (when the stream is not
// being captured; otherwise the heuristic's first), with L2 flushed before
// each timed run for shapes of at most 256 rows.  rocBLAS runs the shapes
// hipBLASLt has no algorithm for.
#pragma once

#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <cstdint>
#include <vector>

#include "common.hpp"

namespace gdn2 {

class Gemm {
  public:
    gdn2_status init();
    void destroy();
    // op(A) [M, Kd]: A stored [M, Kd] (ta = false) or [Kd, M] (ta = true), row stride lda;
    // op(B) [Kd, N]: B stored [Kd, N] (tb = false) or [N, Kd] (tb = true), row stride ldb.
    gdn2_status run(bool ta, bool tb, int64_t M, int64_t N, int64_t Kd, const float *A, int64_t lda, const float *B,
                    int64_t ldb, float *C, int64_t ldc, float beta, hipStream_t s);

  private:
    struct Plan {
        bool ta, tb;
        int64_t M, N, Kd, lda, ldb, ldc;
        bool ok;  // false: hipBLASLt offers no algorithm, use rocBLAS
        hipblasLtMatmulDesc_t desc;
        hipblasLtMatrixLayout_t la, lb, lc;
        hipblasLtMatmulAlgo_t algo;
        size_t ws;
    };
    gdn2_status plan(bool ta, bool tb, int64_t M, int64_t N, int64_t Kd, const float *A, int64_t lda, const float *B,
                     int64_t ldb, int64_t ldc, hipStream_t s, const Plan **out);
    gdn2_status ensure_ws(size_t bytes);
    hipblasLtHandle_t lt_ = nullptr;
    rocblas_handle rb_ = nullptr;
    std::vector<Plan> plans_;
    void *ws_ = nullptr;
    size_t ws_bytes_ = 0;
};

}  // namespace gdn2
