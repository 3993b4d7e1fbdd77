// Deterministic embedding backward (the scatter of alodlm/model.py:133,149 and
// of the re-embedding at model.py:150-151): dtable[id] += sum of dout over the
// rows with that id, every sum in a fixed order.
//
// A plan is built once per id array (one workgroup): a stable LSD radix sort of
// (id, row) on 5-bit digits (ids outside [0, vocab) take the key vocab and
// receive no gradient), the runs of equal ids, and the runs cut into chunks of
// at most EP_CHUNK sorted rows.  The scatter then sums each chunk's rows in
// row order (one workgroup per chunk); a run of one chunk adds its sum to its
// table row directly (the only writer of that row in the launch), longer runs
// (the mask token's rows, frequent tokens) write per-chunk partials that a
// second launch adds up in chunk order.  The same plan serves every filter of
// the rows (rows failing `row_exits[r] <= max_exit` contribute nothing).
#include "embed.h"

#define EP_THREADS 1024
#define EP_CHUNK 32
#define EP_BITS 5
#define EP_BUCKETS 32
#define EP_HEADER 8
// one workgroup of 256 threads per chunk, at most rows chunks: rows * 256 < 2^32
#define EP_MAX_ROWS (1ll << 24)

namespace {

// Plan layout (int32): header [nruns, nchunks, nslots, nmulti, 0...] then
// arrays of n entries.
struct Plan {
  int32_t *hdr, *key, *row, *cbeg, *cend, *crun, *cslot, *rstart, *rfirst, *mbeg, *mend, *mkey,
      *tkey, *trow;
};

__device__ __forceinline__ Plan plan_view(int32_t* base, int64_t n) {
  Plan p;
  p.hdr = base;
  int32_t* a = base + EP_HEADER;
  p.key = a; a += n;
  p.row = a; a += n;
  p.cbeg = a; a += n;
  p.cend = a; a += n;
  p.crun = a; a += n;
  p.cslot = a; a += n;
  p.rstart = a; a += n;
  p.rfirst = a; a += n;
  p.mbeg = a; a += n;
  p.mend = a; a += n;
  p.mkey = a; a += n;
  p.tkey = a; a += n;
  p.trow = a;
  return p;
}

constexpr int64_t kPlanArrays = 13;

// Exclusive scan of one value per thread over the workgroup; *total gets the sum.
__device__ __forceinline__ int block_scan(int v, int* total, int* waves) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) waves[wave] = x;
  __syncthreads();
  int before = 0, sum = 0;
  for (int w = 0; w < EP_THREADS / 64; ++w) {
    if (w < wave) before += waves[w];
    sum += waves[w];
  }
  __syncthreads();
  *total = sum;
  return before + x - v;
}

__device__ __forceinline__ void thread_range(int64_t count, int64_t& lo, int64_t& hi) {
  const int64_t per = (count + EP_THREADS - 1) / EP_THREADS;
  lo = (int64_t)threadIdx.x * per;
  lo = lo < count ? lo : count;
  hi = lo + per < count ? lo + per : count;
}

__global__ void __launch_bounds__(EP_THREADS)
embed_plan_kernel(const int64_t* __restrict__ ids, int64_t n, int64_t vocab, int passes,
                  int32_t* __restrict__ plan) {
  __shared__ uint32_t hist[EP_BUCKETS][EP_THREADS];  // 128 KB
  __shared__ int waves[EP_THREADS / 64];
  Plan P = plan_view(plan, n);
  const int t = threadIdx.x;
  int64_t lo, hi;
  thread_range(n, lo, hi);
  for (int64_t i = lo; i < hi; ++i) {
    const int64_t id = ids[i];
    P.key[i] = (id >= 0 && id < vocab) ? (int32_t)id : (int32_t)vocab;
    P.row[i] = (int32_t)i;
  }
  __syncthreads();
  // ---- stable LSD radix sort: each thread owns a contiguous range, so thread
  // order is element order and the (digit, thread)-major offsets keep it
  int32_t *ks = P.key, *rs = P.row, *kd = P.tkey, *rd = P.trow;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = pass * EP_BITS;
    for (int d = 0; d < EP_BUCKETS; ++d) hist[d][t] = 0;
    for (int64_t i = lo; i < hi; ++i) hist[(ks[i] >> shift) & (EP_BUCKETS - 1)][t] += 1;
    __syncthreads();
    {
      // flattened index f = d * EP_THREADS + thread; this thread scans
      // f in [32 t, 32 t + 32), i.e. digit t / 32, threads 32 (t % 32) ...
      const int d = t >> 5, t0 = (t & 31) * 32;
      int s = 0;
      for (int k = 0; k < 32; ++k) s += (int)hist[d][t0 + k];
      int total;
      int base = block_scan(s, &total, waves);
      for (int k = 0; k < 32; ++k) {
        const int c = (int)hist[d][t0 + k];
        hist[d][t0 + k] = (uint32_t)base;
        base += c;
      }
    }
    __syncthreads();
    for (int64_t i = lo; i < hi; ++i) {
      const int32_t k = ks[i];
      const uint32_t pos = hist[(k >> shift) & (EP_BUCKETS - 1)][t]++;
      kd[pos] = k;
      rd[pos] = rs[i];
    }
    __syncthreads();
    int32_t* tmp = ks; ks = kd; kd = tmp;
    tmp = rs; rs = rd; rd = tmp;
  }
  if (ks != P.key) {  // an odd number of passes left the result in the scratch pair
    for (int64_t i = lo; i < hi; ++i) { P.key[i] = ks[i]; P.row[i] = rs[i]; }
    __syncthreads();
  }
  // ---- runs of equal keys: rstart[r]; the run of every position goes to
  // cslot (scratch) for the chunk pass
  int cnt = 0;
  for (int64_t i = lo; i < hi; ++i) cnt += (i == 0 || P.key[i] != P.key[i - 1]);
  int nruns;
  int r = block_scan(cnt, &nruns, waves) - 1;
  for (int64_t i = lo; i < hi; ++i) {
    if (i == 0 || P.key[i] != P.key[i - 1]) P.rstart[++r] = (int32_t)i;
    P.cslot[i] = r;
  }
  __syncthreads();
  // ---- chunks: a new chunk at every run start and every EP_CHUNK rows of a run
  cnt = 0;
  for (int64_t i = lo; i < hi; ++i) cnt += ((i - P.rstart[P.cslot[i]]) % EP_CHUNK) == 0;
  int nchunks;
  int c = block_scan(cnt, &nchunks, waves) - 1;
  for (int64_t i = lo; i < hi; ++i) {
    const int32_t run = P.cslot[i];
    const int64_t pos = i - P.rstart[run];
    if (pos % EP_CHUNK == 0) {
      P.cbeg[++c] = (int32_t)i;
      P.crun[c] = run;
      if (pos == 0) P.rfirst[run] = c;
    }
  }
  __syncthreads();
  // ---- chunk ends; partial slots of the chunks of multi-chunk runs (in
  // chunk order, so a run's slots are consecutive)
  int64_t clo, chi;
  thread_range(nchunks, clo, chi);
  cnt = 0;
  for (int64_t k = clo; k < chi; ++k) {
    P.cend[k] = k + 1 < nchunks ? P.cbeg[k + 1] : (int32_t)n;
    const int32_t run = P.crun[k];
    const int32_t rend = run + 1 < nruns ? P.rstart[run + 1] : (int32_t)n;
    cnt += (rend - P.rstart[run]) > EP_CHUNK;
  }
  int nslots;
  int slot = block_scan(cnt, &nslots, waves);
  for (int64_t k = clo; k < chi; ++k) {
    const int32_t run = P.crun[k];
    const int32_t rend = run + 1 < nruns ? P.rstart[run + 1] : (int32_t)n;
    P.cslot[k] = (rend - P.rstart[run]) > EP_CHUNK ? slot++ : -1;
  }
  __syncthreads();
  // ---- multi-chunk runs: the range of their partial slots
  int64_t rlo, rhi;
  thread_range(nruns, rlo, rhi);
  cnt = 0;
  for (int64_t q = rlo; q < rhi; ++q) {
    const int32_t rend = q + 1 < nruns ? P.rstart[q + 1] : (int32_t)n;
    cnt += (rend - P.rstart[q]) > EP_CHUNK;
  }
  int nmulti;
  int m = block_scan(cnt, &nmulti, waves);
  for (int64_t q = rlo; q < rhi; ++q) {
    const int32_t rend = q + 1 < nruns ? P.rstart[q + 1] : (int32_t)n;
    const int32_t len = rend - P.rstart[q];
    if (len > EP_CHUNK) {
      const int32_t first = P.cslot[P.rfirst[q]];
      P.mbeg[m] = first;
      P.mend[m] = first + (len + EP_CHUNK - 1) / EP_CHUNK;
      P.mkey[m] = P.key[P.rstart[q]];
      ++m;
    }
  }
  if (t == 0) {
    P.hdr[0] = nruns;
    P.hdr[1] = nchunks;
    P.hdr[2] = nslots;
    P.hdr[3] = nmulti;
  }
}

// One workgroup per chunk (grid.x: an upper bound, extra groups exit), W
// columns per thread (8 with 16-byte loads when hidden % 8 == 0).
template <typename T, int W>
__global__ void __launch_bounds__(256)
embed_chunk_kernel(const T* __restrict__ dout, const int32_t* __restrict__ plan, int64_t n,
                   const int32_t* __restrict__ row_exits, int64_t max_exit,
                   float* __restrict__ dtable, float* __restrict__ partial, int64_t H,
                   int64_t vocab, int64_t max_slots) {
  Plan P = plan_view(const_cast<int32_t*>(plan), n);
  const int64_t c = blockIdx.x;
  if (c >= P.hdr[1]) return;
  const int64_t col = ((int64_t)blockIdx.y * 256 + threadIdx.x) * W;
  if (col >= H) return;
  const int32_t b = P.cbeg[c], e = P.cend[c];
  if (b < 0 || b >= e || e > n) return;  // the plan is built in range; never read past it
  const int32_t key = P.key[b];
  if (key < 0 || key >= vocab) return;
  float acc[W];
#pragma unroll
  for (int i = 0; i < W; ++i) acc[i] = 0.f;
  bool any = false;
  for (int32_t p = b; p < e; ++p) {
    const int64_t r = P.row[p];
    if (r < 0 || r >= n || (row_exits && row_exits[r] > max_exit)) continue;
    any = true;
    if constexpr (W == 8) {
      float v[8];
      Vec8<T>::load(dout + r * H + col, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += v[i];
    } else {
      acc[0] += Elem<T>::load(dout, r * H + col);
    }
  }
  const int32_t slot = P.cslot[c];
  if (slot >= max_slots) return;
  if (slot >= 0) {  // a chunk of a long run: its partial, zero when every row was filtered
    float* dst = partial + (int64_t)slot * H + col;
    if constexpr (W == 8) Vec8<float>::store(dst, acc);
    else dst[0] = acc[0];
  } else if (any) {  // the run's only chunk: the only writer of this table row
    float* dst = dtable + (int64_t)key * H + col;
    if constexpr (W == 8) {
      float cur[8];
      Vec8<float>::load(dst, cur);
#pragma unroll
      for (int i = 0; i < 8; ++i) cur[i] += acc[i];
      Vec8<float>::store(dst, cur);
    } else {
      dst[0] += acc[0];
    }
  }
}

__global__ void __launch_bounds__(256)
embed_run_kernel(const int32_t* __restrict__ plan, int64_t n, float* __restrict__ dtable,
                 const float* __restrict__ partial, int64_t H, int64_t vocab, int64_t max_slots) {
  Plan P = plan_view(const_cast<int32_t*>(plan), n);
  const int64_t m = blockIdx.x;
  if (m >= P.hdr[3]) return;
  const int64_t col = (int64_t)blockIdx.y * 256 + threadIdx.x;
  if (col >= H) return;
  const int32_t key = P.mkey[m];
  const int32_t s0 = P.mbeg[m], s1 = P.mend[m];
  if (key < 0 || key >= vocab || s0 < 0 || s1 > max_slots) return;
  float acc = 0.f;
  for (int32_t s = s0; s < s1; ++s) acc += partial[(int64_t)s * H + col];
  dtable[(int64_t)key * H + col] += acc;
}

}  // namespace

extern "C" int64_t alodlm_embed_plan_size(int64_t rows) { return EP_HEADER + kPlanArrays * rows; }

extern "C" int alodlm_embed_plan(const int64_t* ids, int64_t rows, int64_t vocab, int32_t* plan,
                                 void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && rows < EP_MAX_ROWS, "embed_plan: rows out of range");
  ALODLM_CHECK_ARG(vocab > 0 && vocab < (1ll << 30), "embed_plan: vocab out of range");
  if (rows == 0) return ALODLM_OK;
  int bits = 1;
  while ((1ll << bits) <= vocab) ++bits;  // keys 0..vocab
  const int passes = (bits + EP_BITS - 1) / EP_BITS;
  embed_plan_kernel<<<1, EP_THREADS, 0, as_stream(stream)>>>(ids, rows, vocab, passes, plan);
  ALODLM_CHECK_LAUNCH("embed_plan");
  return ALODLM_OK;
}

extern "C" int64_t alodlm_embed_scatter_workspace(int64_t rows, int64_t hidden) {
  // partial slots: a run of L > EP_CHUNK rows takes ceil(L / EP_CHUNK) <= 2 L / EP_CHUNK
  return (2 * rows / EP_CHUNK + 1) * hidden;
}

int embed_scatter_launch(const void* dout, const int32_t* plan, const int32_t* row_exits,
                         int64_t max_exit, float* dtable, float* workspace, int64_t rows,
                         int64_t hidden, int64_t vocab, int dtype, hipStream_t st) {
  ALODLM_CHECK_ARG(rows >= 0 && rows < EP_MAX_ROWS && hidden > 0,
                   "embed_scatter_add: bad shape");
  if (rows == 0) return ALODLM_OK;
  const int64_t max_slots = alodlm_embed_scatter_workspace(rows, hidden) / hidden;
  const bool v8 = hidden % 8 == 0 && aligned8(dout, dtype) &&
                  reinterpret_cast<uintptr_t>(dtable) % 32 == 0 &&
                  reinterpret_cast<uintptr_t>(workspace) % 32 == 0;
  ALODLM_DISPATCH(dtype, T, {
    if (v8)
      embed_chunk_kernel<T, 8><<<dim3((unsigned)rows, ceil_div_u(hidden, 256 * 8)), 256, 0, st>>>(
          (const T*)dout, plan, rows, row_exits, max_exit, dtable, workspace, hidden, vocab,
          max_slots);
    else
      embed_chunk_kernel<T, 1><<<dim3((unsigned)rows, ceil_div_u(hidden, 256)), 256, 0, st>>>(
          (const T*)dout, plan, rows, row_exits, max_exit, dtable, workspace, hidden, vocab,
          max_slots);
  });
  ALODLM_CHECK_LAUNCH("embed_scatter_chunks");
  embed_run_kernel<<<dim3((unsigned)(rows / (EP_CHUNK + 1) + 1), ceil_div_u(hidden, 256)), 256, 0,
                     st>>>(plan, rows, dtable, workspace, hidden, vocab, max_slots);
  ALODLM_CHECK_LAUNCH("embed_scatter_runs");
  return ALODLM_OK;
}

extern "C" int alodlm_embed_scatter_add(const void* dout, const int32_t* plan,
                                        const int32_t* row_exits, int64_t max_exit, float* dtable,
                                        float* workspace, int64_t rows, int64_t hidden,
                                        int64_t vocab, int dtype, void* stream) {
  return embed_scatter_launch(dout, plan, row_exits, max_exit, dtable, workspace, rows, hidden,
                              vocab, dtype, as_stream(stream));
}
