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
