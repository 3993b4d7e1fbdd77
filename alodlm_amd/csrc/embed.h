// The deterministic embedding scatter shared with the carry-select backward.
#pragma once

#include "common.h"

// dtable[key] += sum of dout rows in the plan's order (rows with row_exits ==
// NULL or row_exits[r] <= max_exit).  `workspace` holds
// alodlm_embed_scatter_workspace(rows, hidden) floats.
int embed_scatter_launch(const void* dout, const int32_t* plan, const int32_t* row_exits,
                         int64_t max_exit, float* dtable, float* workspace, int64_t rows,
                         int64_t hidden, int64_t vocab, int dtype, hipStream_t st);
