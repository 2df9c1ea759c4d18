// gemm_lib.hpp -- hipBLASLt state of a backend and the plain bf16 GEMM the
// graph executor runs through it (gemm_lib.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dit {

struct LtState;

// A handle and a 32 MiB workspace; DT_OK or a DT_ERR_* code.
int lt_create(LtState** out);
void lt_destroy(LtState* st);

// DT_ERR_INVALID_ARG, naming `what`, when `stream` is being captured: the
// handle and the per-shape plans are made outside captures, so that a
// captured graph holds only the GEMM launches.
int lt_refuse_under_capture(hipStream_t stream, const char* what);

// C[M][N] = A[M][K] . B[N][K]^T (+ addend[M][N] with row stride ldd), bf16
// operands, fp32 accumulation, output of out_type (F32 or BF16).
int lt_gemm(LtState* st, hipStream_t stream, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
            int64_t ldc, int64_t M, int64_t N, int64_t K, const void* addend, int64_t ldd, int32_t out_type);

}  // namespace dit
