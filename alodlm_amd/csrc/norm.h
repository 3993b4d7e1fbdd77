// Internal helpers shared between the norm-family translation units.
#pragma once

#include "common.h"

// Group sums the column reduction keeps in its scratch (at most this many rows).
#define COLUMN_REDUCE_MAX_GROUPS 64

// out[c] += sum_p partial[p * ld + col0 + c] for c < ncols (deterministic order).
// `tmp` holds COLUMN_REDUCE_MAX_GROUPS * ncols floats of scratch, disjoint from
// `partial`.
int column_reduce(const float* partial, int64_t nparts, int64_t ld, int64_t col0, int64_t ncols,
                  float* out, float* tmp, hipStream_t st);

// Rows per block of the backward kernels that write one partial row of
// weight-gradient sums per block: 32 for large row counts, fewer (a multiple
// of 4, at least 4) so that about 512 blocks keep every CU busy when rows are
// few (the 8B step's 4096-row packs).
static inline int64_t bwd_rows_per_block(int64_t rows) {
  int64_t r = (rows + 511) / 512;
  r = (r + 3) / 4 * 4;
  return r < 4 ? 4 : (r > 32 ? 32 : r);
}

// RMSNorm backward (and the carry-norm backward when skip_exits is set: rows
// with skip_exits[r] <= skip_depth pass dres through).  `workspace` holds
// alodlm_rmsnorm_bwd_workspace(rows, cols) floats; every element of it the
// launch reads is written earlier in the same launch sequence.
int rmsnorm_bwd_launch(const void* dy, const void* x, const float* rstd, const void* w,
                       const void* dres, void* dx, float* dw_accum, float* workspace,
                       int64_t rows, int64_t cols, int dtype, const int32_t* skip_exits,
                       int64_t skip_depth, hipStream_t st);
