// Internal helpers shared between the norm-family translation units.
#pragma once

#include "common.h"

// out[c] += sum_p partial[p * ld + col0 + c] for c < ncols (deterministic order).
int column_reduce(const float* partial, int64_t nparts, int64_t ld, int64_t col0, int64_t ncols,
                  float* out, hipStream_t st);
