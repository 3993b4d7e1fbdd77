// Dual-stream batch construction (alodlm/batch.py:34-85).
//
// Integer work only: every output is bit-exact with the reference given the
// same draws.  One thread owns one masking block; the block's chosen flags sit
// in LDS.  The per-block work is tiny (block_size <= 1024 tokens), the launch
// covers every block of the pack at once.
#include "common.h"

#define BATCH_THREADS 64

__global__ void __launch_bounds__(BATCH_THREADS)
batch_build_kernel(const int64_t* __restrict__ ids, const int64_t* __restrict__ labels,
                   const int64_t* __restrict__ seg, const int32_t* __restrict__ seg_block,
                   int64_t n_segments, int64_t n_blocks, int64_t B, int64_t mask_token,
                   const float* __restrict__ block_p, const int32_t* __restrict__ block_count,
                   const int64_t* __restrict__ perm_offset, const int64_t* __restrict__ perms,
                   int64_t* __restrict__ out_ids, int64_t* __restrict__ out_original,
                   int64_t* __restrict__ out_positions, uint8_t* __restrict__ out_masked,
                   float* __restrict__ out_prob, int32_t* __restrict__ row_segment,
                   int32_t* __restrict__ ar_target) {
  extern __shared__ unsigned char lds_flags[];
  const int64_t blk = (int64_t)blockIdx.x * BATCH_THREADS + threadIdx.x;
  if (blk >= n_blocks) return;
  unsigned char* chosen = lds_flags + (int64_t)threadIdx.x * B;
  // segment of this block: seg_block is nondecreasing with seg_block[0] = 0
  int64_t lo = 0, hi = n_segments;  // find s with seg_block[s] <= blk < seg_block[s+1]
  while (hi - lo > 1) {
    int64_t mid = (lo + hi) >> 1;
    if (seg_block[mid] <= blk) lo = mid; else hi = mid;
  }
  const int64_t s = lo;
  const int64_t a = seg[s];
  const int64_t L = seg[s + 1] - a;
  const int64_t b = blk - seg_block[s];
  const int64_t left = b * B;
  const int64_t right = left + B < L ? left + B : L;
  const int64_t width = right - left;
  for (int64_t j = 0; j < width; ++j) chosen[j] = 0;
  // chosen[candidate[perm[:count]]] = True  (batch.py:55-60)
  const int32_t count = block_count[blk];
  if (count > 0) {
    const int64_t* perm = perms + perm_offset[blk];
    for (int32_t t = 0; t < count; ++t) {
      // perm[t]-th candidate (label != -100) of the block, in ascending order
      int64_t want = perm[t], seen = 0;
      for (int64_t j = 0; j < width; ++j) {
        if (labels[a + left + j] != -100) {
          if (seen == want) { chosen[j] = 1; break; }
          ++seen;
        }
      }
    }
  }
  const float p = block_p[blk];
  // clean stream: the segment's tokens at positions 0..L-1, never masked
  const int64_t clean = 2 * a;
  const int64_t noisy = 2 * a + L;
  for (int64_t j = left; j < right; ++j) {
    out_ids[clean + j] = ids[a + j];
    out_original[clean + j] = ids[a + j];
    out_positions[clean + j] = j;
    out_masked[clean + j] = 0;
    out_prob[clean + j] = 0.f;
    row_segment[clean + j] = (int32_t)s;
    row_segment[noisy + j] = (int32_t)s;
    // next-token target of clean row j (alodlm/loss.py:20-25): labels[a+j+1]
    const int64_t next = j + 1 < L ? labels[a + j + 1] : -100;
    ar_target[clean + j] = next == -100 ? -1 : (int32_t)next;
    ar_target[noisy + j] = -1;
  }
  // noisy stream: observed tokens first, then masked ones, each ascending
  int64_t o = noisy + left;
  for (int pass = 0; pass < 2; ++pass) {
    for (int64_t j = 0; j < width; ++j) {
      if (chosen[j] != pass) continue;
      const int64_t tok = ids[a + left + j];
      out_ids[o] = pass ? mask_token : tok;
      out_original[o] = tok;
      out_positions[o] = left + j;
      out_masked[o] = (uint8_t)pass;
      out_prob[o] = pass ? p : 0.f;
      ++o;
    }
  }
}

__global__ void batch_bounds_kernel(const int64_t* seg, int64_t n_segments, int64_t* out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= n_segments) out[i] = 2 * seg[i];
}

extern "C" int alodlm_batch_build(const int64_t* ids, const int64_t* labels, const int64_t* seg,
                                  const int32_t* seg_block, int64_t n_segments, int64_t n_blocks,
                                  int64_t block_size, int64_t mask_token_id, const float* block_p,
                                  const int32_t* block_count, const int64_t* perm_offset,
                                  const int64_t* perms, int64_t* out_ids, int64_t* out_original,
                                  int64_t* out_positions, uint8_t* out_masked, float* out_prob,
                                  int32_t* row_segment, int32_t* ar_target,
                                  int64_t* out_boundaries, void* stream) {
  ALODLM_CHECK_ARG(n_segments >= 1 && n_blocks >= 1, "batch_build: empty pack");
  ALODLM_CHECK_ARG(block_size >= 1 && block_size <= 1024, "batch_build: block_size must be in [1, 1024]");
  hipStream_t st = as_stream(stream);
  size_t lds = (size_t)BATCH_THREADS * (size_t)block_size;
  batch_build_kernel<<<ceil_div_u(n_blocks, BATCH_THREADS), BATCH_THREADS, lds, st>>>(
      ids, labels, seg, seg_block, n_segments, n_blocks, block_size, mask_token_id, block_p,
      block_count, perm_offset, perms, out_ids, out_original, out_positions, out_masked,
      out_prob, row_segment, ar_target);
  ALODLM_CHECK_LAUNCH("batch_build");
  batch_bounds_kernel<<<ceil_div_u(n_segments + 1, 256), 256, 0, st>>>(seg, n_segments,
                                                                       out_boundaries);
  ALODLM_CHECK_LAUNCH("batch_bounds");
  return ALODLM_OK;
}
