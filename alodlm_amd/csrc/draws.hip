// Masking draws of one pack (alodlm/batch.py:50-60) in two launches instead of
// one uniform_ per segment plus one randperm per masked block.
//
// The reference draws, per segment, ceil(L/B) mask ratios with
// `torch.empty(n).uniform_(0, 1).clamp_min(1e-8)` and then, for every block
// whose masked count round(n_cand * p) is nonzero, `torch.randperm(n_cand)`,
// all from the device's default Philox generator.  The values of those calls
// are fixed by the generator's (seed, offset) when they are made, and the
// offset each call consumes is fixed by its size, so the whole sequence can be
// evaluated here from the (seed, offset) the generator holds on entry:
//
//   uniform_ of n floats (ATen/native/cuda/DistributionTemplates.h,
//     distribution_elementwise_grid_stride_kernel + calc_execution_policy):
//     element i is the first output of Philox stream (seed, subsequence i,
//     offset), mapped to (0, 1] by 2^-32 + v * 2^-32 and 1.0 reversed to 0;
//     the offset advances by 4.
//   randperm(n), n < 2^31 with at most 32 key bits (the randperm note in
//     ATen/native/cuda/Randperm.cuh): int keys from random_(INT_MIN, INT_MAX)
//     (64-bit draws (x << 32 | y) of stream (seed, i, offset) reduced modulo
//     2^32 - 1; offset += 4), a stable ascending sort of arange(n) by the low
//     `bits` key bits, then every run of equal keys shuffled by Fisher-Yates
//     with stream (seed, run start, offset) (randperm_handle_duplicate_keys;
//     offset += n rounded up to 4).  `bits` is computed on the host exactly as
//     torch does, in double precision, and passed as a table by n.
//
// Philox4x32-10 is the counter-based generator of Salmon, Moraes, Dror and
// Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC 2011).  A stream
// (seed, subsequence, offset) is the cuRAND/rocRAND convention: key = seed,
// counter = (offset / 4, subsequence) as two 64-bit halves, outputs taken four
// at a time from successive counters (offsets here are multiples of 4).
#include "common.h"

namespace {

struct Philox {
  uint32_t c0, c1, c2, c3;  // counter: (c1:c0) = offset / 4, (c3:c2) = subsequence
  uint32_t k0, k1;

  __device__ Philox(uint64_t seed, uint64_t subsequence, uint64_t offset) {
    const uint64_t block = offset >> 2;
    c0 = (uint32_t)block;
    c1 = (uint32_t)(block >> 32);
    c2 = (uint32_t)subsequence;
    c3 = (uint32_t)(subsequence >> 32);
    k0 = (uint32_t)seed;
    k1 = (uint32_t)(seed >> 32);
  }

  // Ten rounds on the current counter; the counter then steps by one.
  __device__ uint4 next4() {
    uint32_t x0 = c0, x1 = c1, x2 = c2, x3 = c3, a = k0, b = k1;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
      const uint64_t m0 = (uint64_t)0xD2511F53u * x0;
      const uint64_t m1 = (uint64_t)0xCD9E8D57u * x2;
      const uint32_t y0 = (uint32_t)(m1 >> 32) ^ x1 ^ a;
      const uint32_t y2 = (uint32_t)(m0 >> 32) ^ x3 ^ b;
      x1 = (uint32_t)m1;
      x3 = (uint32_t)m0;
      x0 = y0;
      x2 = y2;
      a += 0x9E3779B9u;
      b += 0xBB67AE85u;
    }
    if (++c0 == 0 && ++c1 == 0 && ++c2 == 0) ++c3;
    return make_uint4(x0, x1, x2, x3);
  }
};

// Successive 32-bit outputs of one stream (curand() order: x, y, z, w, ...).
struct PhiloxWords {
  Philox g;
  uint4 buf;
  int used;
  __device__ PhiloxWords(uint64_t seed, uint64_t subsequence, uint64_t offset)
      : g(seed, subsequence, offset), used(4) {}
  __device__ uint32_t operator()() {
    if (used == 4) { buf = g.next4(); used = 0; }
    const uint32_t v = used == 0 ? buf.x : used == 1 ? buf.y : used == 2 ? buf.z : buf.w;
    ++used;
    return v;
  }
};

constexpr int RATIO_THREADS = 1024;

// One workgroup walks the segments in order: segment s's ratios come from the
// offset its predecessors leave, and its randperms' offsets follow from its
// masked counts (a prefix sum over its blocks).
__global__ void __launch_bounds__(RATIO_THREADS)
mask_ratio_kernel(uint64_t seed, uint64_t offset, const int32_t* __restrict__ seg_block,
                  int n_segments, const int32_t* __restrict__ block_n, int block_size,
                  float* __restrict__ block_p, int32_t* __restrict__ block_count,
                  uint64_t* __restrict__ block_offset, int64_t* __restrict__ perm_offset,
                  uint64_t* __restrict__ offset_out) {
  __shared__ uint32_t wave_total[RATIO_THREADS / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t base = offset;
  for (int s = 0; s < n_segments; ++s) {
    const int b0 = seg_block[s], nb = seg_block[s + 1] - b0;
    const uint64_t ratio_offset = base;
    uint64_t run = base + 4;  // the first randperm follows the ratios' uniform_
    for (int c = 0; c < nb; c += RATIO_THREADS) {
      const int i = c + (int)threadIdx.x;
      uint32_t cost = 0;
      if (i < nb) {
        const uint32_t v = Philox(seed, (uint64_t)i, ratio_offset).next4().x;
        float u = 0x1p-32f + (float)v * 0x1p-32f;  // the product is exact
        if (u == 1.0f) u = 0.0f;
        const float p = fmaxf(u, 1e-8f);
        const int n = block_n[b0 + i];
        // Python's round of a float64 product: ties to even (rint's default mode)
        const int count = (int)rint((double)n * (double)p);
        block_p[b0 + i] = p;
        block_count[b0 + i] = count;
        perm_offset[b0 + i] = (int64_t)(b0 + i) * block_size;
        cost = count > 0 ? 4u + (((uint32_t)n + 3u) & ~3u) : 0u;
      }
      // exclusive prefix sum of cost over the chunk
      uint32_t incl = cost;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const uint32_t t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
      }
      if (lane == 63) wave_total[wave] = incl;
      __syncthreads();
      uint32_t before = 0, total = 0;
      for (int w = 0; w < RATIO_THREADS / 64; ++w) {
        const uint32_t t = wave_total[w];
        before += w < wave ? t : 0u;
        total += t;
      }
      if (i < nb) block_offset[b0 + i] = run + before + (incl - cost);
      run += total;
      __syncthreads();  // wave_total is rewritten by the next chunk
    }
    base = run;
  }
  if (threadIdx.x == 0) *offset_out = base;
}

constexpr int PERM_MAX = 1024;

// One wavefront per masked block: torch.randperm(n) at the block's offset.
__global__ void __launch_bounds__(64)
block_randperm_kernel(uint64_t seed, const int32_t* __restrict__ block_n,
                      const int32_t* __restrict__ block_count,
                      const uint64_t* __restrict__ block_offset,
                      const int32_t* __restrict__ key_bits, int block_size,
                      int64_t* __restrict__ perms) {
  __shared__ uint32_t key[PERM_MAX];
  __shared__ uint32_t sorted_key[PERM_MAX];
  __shared__ int32_t data[PERM_MAX];
  const int blk = blockIdx.x;
  if (block_count[blk] <= 0) return;  // the whole workgroup leaves together
  const int n = block_n[blk];
  if (n < 1 || n > block_size) return;  // the host passes 1 <= n <= block_size here
  const uint64_t off = block_offset[blk];
  const uint32_t mask = (uint32_t)((1ull << key_bits[n]) - 1ull);
  const int lane = threadIdx.x;
  for (int j = lane; j < n; j += 64) {
    const uint4 r = Philox(seed, (uint64_t)j, off).next4();
    const uint64_t r64 = ((uint64_t)r.x << 32) | r.y;
    // (r64 mod (2^32 - 1)) + INT_MIN as int32; the sort reads bits below 31,
    // which the added INT_MIN leaves alone
    key[j] = (uint32_t)(r64 % 4294967295ull) & mask;
  }
  __syncthreads();
  // stable ascending sort of arange(n) by key: rank = smaller keys + equal
  // keys earlier in the input
  for (int j = lane; j < n; j += 64) {
    const uint32_t k = key[j];
    int rank = 0;
    for (int i = 0; i < n; ++i) {
      const uint32_t ki = key[i];
      rank += (ki < k) || (ki == k && i < j);
    }
    sorted_key[rank] = k;
    data[rank] = j;
  }
  __syncthreads();
  // runs of equal keys: the run's first position shuffles it (Fisher-Yates)
  const uint64_t dup_offset = off + 4;
  for (int t = lane; t < n - 1; t += 64) {
    const uint32_t k = sorted_key[t];
    if (sorted_key[t + 1] != k) continue;
    if (t != 0 && sorted_key[t - 1] == k) continue;
    int size = 2;
    while (t + size < n && sorted_key[t + size] == k) ++size;
    PhiloxWords words(seed, (uint64_t)t, dup_offset);
    for (int i = size - 1; i > 0; --i) {
      const int r = (int)(words() % (uint32_t)(i + 1));
      if (r != i) {
        const int32_t tmp = data[t + i];
        data[t + i] = data[t + r];
        data[t + r] = tmp;
      }
    }
  }
  __syncthreads();
  int64_t* out = perms + (int64_t)blk * block_size;
  for (int j = lane; j < n; j += 64) out[j] = data[j];
}

}  // namespace

extern "C" int alodlm_mask_draws(uint64_t seed, uint64_t offset, const int32_t* seg_block,
                                 int64_t n_segments, const int32_t* block_n, int64_t n_blocks,
                                 int64_t block_size, const int32_t* key_bits, float* block_p,
                                 int32_t* block_count, uint64_t* block_offset,
                                 int64_t* perm_offset, int64_t* perms, uint64_t* offset_out,
                                 void* stream) {
  ALODLM_CHECK_ARG(n_segments >= 1 && n_blocks >= 1, "mask_draws: empty pack");
  ALODLM_CHECK_ARG(n_blocks < (1ll << 24), "mask_draws: %lld blocks is too many",
                   (long long)n_blocks);
  ALODLM_CHECK_ARG(block_size >= 1 && block_size <= PERM_MAX,
                   "mask_draws: block_size must be in [1, %d]", PERM_MAX);
  ALODLM_CHECK_ARG(offset % 4 == 0, "mask_draws: generator offset %llu is not a multiple of 4",
                   (unsigned long long)offset);
  hipStream_t st = as_stream(stream);
  mask_ratio_kernel<<<1, RATIO_THREADS, 0, st>>>(seed, offset, seg_block, (int)n_segments,
                                                 block_n, (int)block_size, block_p, block_count,
                                                 block_offset, perm_offset, offset_out);
  ALODLM_CHECK_LAUNCH("mask_ratio");
  block_randperm_kernel<<<(unsigned)n_blocks, 64, 0, st>>>(seed, block_n, block_count,
                                                           block_offset, key_bits,
                                                           (int)block_size, perms);
  ALODLM_CHECK_LAUNCH("block_randperm");
  return ALODLM_OK;
}
