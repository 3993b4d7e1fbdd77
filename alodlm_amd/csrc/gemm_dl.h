// The direct-load GEMM (gemm_dl.hip) as the other GEMM sources call it.
#pragma once

#include "common.h"

// K taken from up to 8 segments with their own operand bases: segment i holds
// k rows [i * k, (i + 1) * k) of both operands (m/n-contiguous operands, one
// leading dimension each), so that one product sums A_i^T B_i over separate
// buffers.  The workgroup's tile walk switches base where a segment ends.
constexpr int KSEGS_MAX = 8;
struct KSegs {
  const bf16_t* a[KSEGS_MAX];
  const bf16_t* b[KSEGS_MAX];
  int64_t k;
};

bool gemm_dl_eligible(int64_t lda, int a_kmajor, int64_t ldb, int b_kmajor, int64_t M, int64_t N,
                      int64_t K);
int64_t gemm_dl_splits(int64_t M, int64_t N, int64_t K);
int64_t gemm_dl_store_splits(int64_t M, int64_t N, int64_t K);
// `segs` (or nullptr): K over separate segments, for m/n-contiguous operands
// and the float-output epilogues only
void gemm_dl_launch(const bf16_t* A, int64_t lda, int a_kmajor, const bf16_t* B, int64_t ldb,
                    int b_kmajor, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                    int64_t N, int64_t K, float alpha, int epi, float* part, int64_t splits,
                    int64_t* nsplit_out, int first_into_c, hipStream_t st,
                    const KSegs* segs = nullptr);
