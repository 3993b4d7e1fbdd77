// Window bookkeeping of adaptive recurrent decoding on the device.
//
// The decoding rules are those of alodlm/inference.py:71-246; the state they
// act on lives in device arrays (alodlm_decode_state) instead of host lists:
//
//  * the ledger: the pending tail of the generated text in logical order, one
//    slot per position, open (still a mask token) or committed (token, exit
//    depth, first-pass halt probability);
//  * the output stream of retired tokens;
//  * the current window: its rows (committed slots first, then open slots,
//    each group in logical order), their token ids and rotary positions, and
//    per mask row the survival, the committed token and its depth;
//  * an int64 header the host reads once per executed depth.
//
// One workgroup runs each kernel: the work is a few thousand slots at most
// and sits between the layer launches of a window.  At the depth where a
// window stops, the commit kernel also retires the window (the committed run
// at the ledger's start is emitted and becomes cache rows, the window's
// commitments are written back to their slots) and plans the next window, so
// the host learns the outcome of a depth and the shape of the next window
// from one header read.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

struct Shared {
  int64_t hdr[ALODLM_DECODE_HEADER];
  int ired[kWaves];
  double dred[kWaves];
};

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = min(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ int block_min_i(int v, Shared& sh) {
  v = wave_min_i(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.ired[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = sh.ired[0];
  for (int w = 1; w < kWaves; ++w) r = min(r, sh.ired[w]);
  return r;
}
__device__ int block_sum_i(int v, Shared& sh) {
  v = wave_sum_i(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.ired[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
  for (int w = 0; w < kWaves; ++w) r += sh.ired[w];
  return r;
}
__device__ double block_sum_d(double v, Shared& sh) {
  v = wave_sum_d(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.dred[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0.0;
  for (int w = 0; w < kWaves; ++w) r += sh.dred[w];
  return r;
}

// Exclusive prefix sum of one int per thread over the block; *total gets the
// block's sum.
__device__ int block_scan_i(int v, int* total, Shared& sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(incl, off, 64);
    if (lane >= off) incl += t;
  }
  __syncthreads();
  if (lane == 63) sh.ired[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) before += sh.ired[w];
    all += sh.ired[w];
  }
  *total = all;
  return before + incl - v;
}

__device__ __forceinline__ bool is_stop(const alodlm_decode_state& s, int64_t token) {
  for (int64_t i = 0; i < s.n_stop; ++i)
    if (s.stop_ids[i] == token) return true;
  return false;
}

// Fresh per-mask-row state and carry tables for a window of `rows` rows of
// which `count` are mask rows.
__device__ void reset_window(const alodlm_decode_state& s, int64_t rows, int64_t count) {
  for (int64_t r = threadIdx.x; r < rows; r += kThreads) s.replace_depth[r] = (int32_t)s.max_depth;
  for (int64_t j = threadIdx.x; j < count; j += kThreads) {
    s.mask_token[j] = 0;
    s.mask_exit[j] = 0;
    s.mask_committed[j] = 0;
    s.mask_fresh[j] = 0;
    s.mask_survival[j] = 1.f;
    s.mask_first_hazard[j] = 0.f;
  }
}

// The top of the decoding loop (alodlm/inference.py:185-210): stop when the
// budget is used, when the committed run at the ledger's start would exceed
// it or holds a stop token (emitting the run up to the stop token), else grow
// the ledger with mask slots to the window size and lay out the window.
__device__ void plan_window(const alodlm_decode_state& s, Shared& sh) {
  const int tid = threadIdx.x;
  int64_t* h = sh.hdr;
  const int64_t n = h[ALODLM_DECODE_LEDGER], gen = h[ALODLM_DECODE_GENERATED];
  const int64_t cache = h[ALODLM_DECODE_CACHE];
  __syncthreads();
  if (gen >= s.max_new_tokens) {
    if (tid == 0) {
      h[ALODLM_DECODE_DONE] = 1;
      h[ALODLM_DECODE_REASON] = ALODLM_DECODE_LENGTH;
      h[ALODLM_DECODE_WINDOW] = 0;
    }
    __syncthreads();
    return;
  }
  // committed run at the start: the first open slot
  int first_open = (int)n;
  for (int64_t i = tid; i < n; i += kThreads)
    if (s.slot_open[i]) { first_open = (int)i; break; }
  const int p = block_min_i(first_open, sh);
  int first_stop = p;
  for (int64_t i = tid; i < p; i += kThreads)
    if (is_stop(s, s.slot_token[i])) { first_stop = (int)i; break; }
  const int stop_at = block_min_i(first_stop, sh);
  if (gen + p >= s.max_new_tokens || stop_at < p) {
    for (int64_t i = tid; i < stop_at; i += kThreads) {
      s.out_token[gen + i] = s.slot_token[i];
      s.out_depth[gen + i] = s.slot_depth[i];
      s.out_halt[gen + i] = s.slot_halt[i];
    }
    __syncthreads();
    if (tid == 0) {
      h[ALODLM_DECODE_GENERATED] = gen + stop_at;
      h[ALODLM_DECODE_DONE] = 1;
      h[ALODLM_DECODE_REASON] = stop_at < p ? ALODLM_DECODE_EOS : ALODLM_DECODE_LENGTH;
      h[ALODLM_DECODE_WINDOW] = 0;
    }
    __syncthreads();
    return;
  }
  const int64_t room = s.max_new_tokens - gen - p;
  const int64_t desired = s.window_size < room ? s.window_size : room;
  const int64_t n2 = n > p + desired ? n : p + desired;
  for (int64_t i = n + tid; i < n2; i += kThreads) {
    s.slot_token[i] = s.mask_token_id;
    s.slot_open[i] = 1;
    s.slot_depth[i] = 0;
    s.slot_halt[i] = 0.f;
  }
  __syncthreads();
  int closed = 0;
  for (int64_t i = tid; i < n2; i += kThreads) closed += s.slot_open[i] ? 0 : 1;
  const int n_obs = block_sum_i(closed, sh);
  // rows: committed slots in logical order, then open slots in logical order;
  // slot p is the first open one (the run before it is committed and the
  // window grows by at least one slot)
  int closed_before = 0, open_before = 0;
  for (int64_t c = 0; c < n2; c += kThreads) {
    const int64_t i = c + tid;
    const bool valid = i < n2;
    const int is_closed = valid && !s.slot_open[i] ? 1 : 0;
    int chunk_closed;
    const int excl = block_scan_i(is_closed, &chunk_closed, sh);
    if (valid) {
      const int64_t token = s.slot_token[i];
      if (is_closed) {
        const int64_t row = closed_before + excl;
        s.row_token[row] = token;
        s.row_position[row] = cache + i;
      } else {
        const int64_t j = open_before + (tid - excl);
        const int64_t row = n_obs + j;
        s.row_token[row] = token;
        s.row_position[row] = cache + i;
        s.mask_row[j] = (int32_t)row;
        s.mask_slot[j] = (int32_t)i;
        s.mask_offset[j] = __fmul_rn((float)(i - p), s.penalty);
      }
    }
    const int64_t in_chunk = n2 - c < kThreads ? n2 - c : kThreads;
    closed_before += chunk_closed;
    open_before += (int)in_chunk - chunk_closed;
  }
  reset_window(s, n2, n2 - n_obs);
  __syncthreads();
  if (tid == 0) {
    h[ALODLM_DECODE_LEDGER] = n2;
    h[ALODLM_DECODE_WINDOW] = n2;
    h[ALODLM_DECODE_OBSERVED] = n_obs;
    h[ALODLM_DECODE_PREFIX] = p;
  }
  __syncthreads();
}

// The end of a window (alodlm/inference.py:227-238): the committed run the
// window started with is emitted and its rows stay in the cache; the
// window's commitments go to their ledger slots; the ledger drops the run.
__device__ void retire_window(const alodlm_decode_state& s, int64_t count, Shared& sh) {
  const int tid = threadIdx.x;
  int64_t* h = sh.hdr;
  const int64_t p = h[ALODLM_DECODE_PREFIX], gen = h[ALODLM_DECODE_GENERATED];
  const int64_t n = h[ALODLM_DECODE_LEDGER];
  for (int64_t i = tid; i < p; i += kThreads) {
    s.out_token[gen + i] = s.slot_token[i];
    s.out_depth[gen + i] = s.slot_depth[i];
    s.out_halt[gen + i] = s.slot_halt[i];
  }
  for (int64_t j = tid; j < count; j += kThreads) {
    if (!s.mask_committed[j]) continue;
    const int32_t slot = s.mask_slot[j];
    s.slot_token[slot] = s.mask_token[j];
    s.slot_open[slot] = 0;
    s.slot_depth[slot] = s.mask_exit[j];
    s.slot_halt[slot] = s.mask_first_hazard[j];
  }
  __syncthreads();
  // move slots [p, n) to [0, n - p), one block-wide chunk at a time (every
  // read of a chunk happens before its writes; later chunks read only slots
  // above everything written so far)
  for (int64_t c = 0; c < n - p; c += kThreads) {
    const int64_t i = c + tid;
    const bool valid = i < n - p;
    int64_t token = 0;
    int32_t open = 0, depth = 0;
    float halt = 0.f;
    if (valid) {
      token = s.slot_token[i + p];
      open = s.slot_open[i + p];
      depth = s.slot_depth[i + p];
      halt = s.slot_halt[i + p];
    }
    __syncthreads();
    if (valid) {
      s.slot_token[i] = token;
      s.slot_open[i] = open;
      s.slot_depth[i] = depth;
      s.slot_halt[i] = halt;
    }
    __syncthreads();
  }
  if (tid == 0) {
    h[ALODLM_DECODE_GENERATED] = gen + p;
    h[ALODLM_DECODE_CACHE] += p;
    h[ALODLM_DECODE_LEDGER] = n - p;
  }
  __syncthreads();
}

__device__ void load_header(const alodlm_decode_state& s, Shared& sh) {
  if (threadIdx.x < ALODLM_DECODE_HEADER) sh.hdr[threadIdx.x] = s.header[threadIdx.x];
  __syncthreads();
}
__device__ void store_header(const alodlm_decode_state& s, Shared& sh) {
  __syncthreads();
  if (threadIdx.x < ALODLM_DECODE_HEADER) s.header[threadIdx.x] = sh.hdr[threadIdx.x];
}

__global__ void __launch_bounds__(kThreads)
decode_plan_kernel(alodlm_decode_state s) {
  __shared__ Shared sh;
  load_header(s, sh);
  plan_window(s, sh);
  store_header(s, sh);
}

__global__ void __launch_bounds__(kThreads)
decode_begin_kernel(alodlm_decode_state s, const int64_t* logical, int64_t rows, int64_t count) {
  reset_window(s, rows, count);
  for (int64_t j = threadIdx.x; j < count; j += kThreads)
    s.mask_offset[j] = __fmul_rn((float)(logical[j] - logical[0]), s.penalty);
}

// One depth's commitments (alodlm/inference.py:109-142): hazards from the
// gate logits of the mask rows, survival, the entropy (or left-to-right)
// agreement, the stop rule with its fallback commitment, and the carry table
// of the next depth; at a stop with `finish`, the window's retirement and the
// next window's plan.
__global__ void __launch_bounds__(kThreads)
decode_commit_kernel(alodlm_decode_state s, const float* __restrict__ gate, int64_t count,
                     int64_t depth, int finish) {
  __shared__ Shared sh;
  const int tid = threadIdx.x;
  load_header(s, sh);
  const int64_t K = s.max_depth;
  int agree_at = -1;  // left1: the first mask row not yet committed
  if (s.mode == ALODLM_DECODE_LEFT1) {
    int first = (int)count;
    for (int64_t j = tid; j < count; j += kThreads)
      if (!s.mask_committed[j]) { first = (int)j; break; }
    agree_at = block_min_i(first, sh);
  }
  int residual = 0, any = 0;
  double unsure = 0.0;
  for (int64_t j = tid; j < count; j += kThreads) {
    const float hazard = sigmoidf_ref(gate[s.mask_row[j]]);
    if (depth == 0) s.mask_first_hazard[j] = hazard;
    const float survival = __fmul_rn(s.mask_survival[j], __fsub_rn(1.f, hazard));
    s.mask_survival[j] = survival;
    const float adjusted = __fadd_rn(s.entropy[j], s.mask_offset[j]);
    const bool was = s.mask_committed[j] != 0;
    const bool agree = s.mode == ALODLM_DECODE_LEFT1 ? j == agree_at : (adjusted < s.tau && !was);
    if (agree) {
      s.mask_token[j] = s.predicted[j];
      s.mask_exit[j] = (int32_t)(depth + 1);
      s.mask_committed[j] = 1;
    }
    s.mask_fresh[j] = agree ? 1 : 0;
    if (was || agree) {
      any = 1;
    } else {
      residual += 1;
      unsure += (double)__fsub_rn(1.f, survival);
    }
  }
  const int n_residual = block_sum_i(residual, sh);
  const int n_any = block_sum_i(any, sh);
  const double total = block_sum_d(unsure, sh);
  const bool stop = depth == K - 1 || n_residual == 0 ||
                    (float)(total / (double)n_residual) >= s.q;
  if (stop && n_any == 0 && count > 0) {
    // nothing committed at a stop: the mask row of least adjusted entropy
    // (the first of equal minima) commits
    float best = INFINITY;
    int best_j = (int)count;
    for (int64_t j = tid; j < count; j += kThreads) {
      const float adjusted = __fadd_rn(s.entropy[j], s.mask_offset[j]);
      if (adjusted < best || (adjusted == best && j < best_j)) { best = adjusted; best_j = (int)j; }
    }
    // block argmin: minimum value, then the smallest index holding it
    __shared__ float fbest[kWaves];
    float v = best;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    __syncthreads();
    if ((tid & 63) == 0) fbest[tid >> 6] = v;
    __syncthreads();
    float m = fbest[0];
    for (int w = 1; w < kWaves; ++w) m = fminf(m, fbest[w]);
    const int pick = block_min_i(best == m ? best_j : (int)count, sh);
    const int j = pick < count ? pick : 0;  // all adjusted NaN: the first row
    if (tid == 0) {
      s.mask_token[j] = s.predicted[j];
      s.mask_exit[j] = (int32_t)(depth + 1);
      s.mask_committed[j] = 1;
    }
  }
  if (!stop) {
    for (int64_t j = tid; j < count; j += kThreads) {
      const int32_t row = s.mask_row[j];
      s.replace_token[row] = s.mask_token[j];
      s.replace_depth[row] = s.mask_fresh[j] ? (int32_t)(depth + 1) : (int32_t)K;
    }
  }
  __syncthreads();
  if (stop && finish) {
    retire_window(s, count, sh);
    plan_window(s, sh);
  }
  // set last: a plan of the next window leaves this field alone
  if (tid == 0) sh.hdr[ALODLM_DECODE_STOP] = stop ? 1 : 0;
  store_header(s, sh);
}

int check_state(const alodlm_decode_state* s) {
  ALODLM_CHECK_ARG(s != nullptr && s->header != nullptr, "decode: no state");
  ALODLM_CHECK_ARG(s->max_depth >= 1, "decode: max_depth must be positive");
  ALODLM_CHECK_ARG(s->n_stop >= 0 && (s->n_stop == 0 || s->stop_ids != nullptr),
                   "decode: bad stop-token list");
  ALODLM_CHECK_ARG(s->mode == ALODLM_DECODE_ENTROPY || s->mode == ALODLM_DECODE_LEFT1,
                   "decode: unknown mode %d", (int)s->mode);
  return ALODLM_OK;
}

}  // namespace

extern "C" int alodlm_decode_plan(const alodlm_decode_state* state, void* stream) {
  const int rc = check_state(state);
  if (rc != ALODLM_OK) return rc;
  ALODLM_CHECK_ARG(state->window_size >= 1 && state->capacity >= 2 * state->window_size,
                   "decode_plan: the ledger needs 2 * window_size slots");
  decode_plan_kernel<<<1, kThreads, 0, as_stream(stream)>>>(*state);
  ALODLM_CHECK_LAUNCH("decode_plan");
  return ALODLM_OK;
}

extern "C" int alodlm_decode_begin(const alodlm_decode_state* state, const int64_t* logical,
                                   int64_t rows, int64_t count, void* stream) {
  const int rc = check_state(state);
  if (rc != ALODLM_OK) return rc;
  ALODLM_CHECK_ARG(rows >= 0 && count >= 0 && count <= rows && rows <= state->capacity,
                   "decode_begin: %lld rows (%lld mask rows) in a state of %lld",
                   (long long)rows, (long long)count, (long long)state->capacity);
  ALODLM_CHECK_ARG(count == 0 || logical != nullptr, "decode_begin: no mask positions");
  decode_begin_kernel<<<1, kThreads, 0, as_stream(stream)>>>(*state, logical, rows, count);
  ALODLM_CHECK_LAUNCH("decode_begin");
  return ALODLM_OK;
}

extern "C" int alodlm_decode_commit(const alodlm_decode_state* state, const float* gate,
                                    int64_t count, int64_t depth, int finish, void* stream) {
  const int rc = check_state(state);
  if (rc != ALODLM_OK) return rc;
  ALODLM_CHECK_ARG(count >= 1 && count <= state->capacity, "decode_commit: %lld mask rows",
                   (long long)count);
  ALODLM_CHECK_ARG(depth >= 0 && depth < state->max_depth, "decode_commit: depth %lld",
                   (long long)depth);
  ALODLM_CHECK_ARG(!finish || state->capacity >= 2 * state->window_size,
                   "decode_commit: the ledger needs 2 * window_size slots");
  decode_commit_kernel<<<1, kThreads, 0, as_stream(stream)>>>(*state, gate, count, depth, finish);
  ALODLM_CHECK_LAUNCH("decode_commit");
  return ALODLM_OK;
}
