// The step objective on [K, rows]: truncated-stick denoising, the sequence
// score-function actor with the geometric prior and the sampled-history
// marginal, the autoregressive mean, the metrics, and d(total)/d(gate)
// (total = (denoising + actor + AR) / 2 for the step; denoising + actor for
// alodlm_outcome_loss, which also writes d(denoising)/d(ce)).
// (alodlm/loss.py:35-90, alodlm/credit.py:7-40, alodlm/model.py:183-187.)
//
// One workgroup of 1024 threads.  Every sum has a fixed order, so the result
// is deterministic.  Segment sums are taken by one wavefront per segment over
// the segment's contiguous rows.
#include "common.h"

#define OBJ_THREADS 1024
#define OBJ_MAX_DEPTH 16

__device__ __forceinline__ void stick_logs(const float* gates, int64_t rows, int64_t r, int K,
                                           float* log_exit) {
  // log_surv[d] = -sum_{j<d} softplus(g[j]); log_exit[d] = log_surv[d] - softplus(-g[d])
  // for d < K-1 and log_surv[K-1] at the final, absorbing depth (loss.py:55-57,64-67).
  float log_surv = 0.f;
  for (int d = 0; d < K; ++d) {
    const float g = gates[(int64_t)d * rows + r];
    log_exit[d] = (d == K - 1) ? log_surv : log_surv - softplusf(-g);
    log_surv -= softplusf(g);
  }
}

__global__ void __launch_bounds__(OBJ_THREADS)
objective_kernel(const float* __restrict__ gates, const int32_t* __restrict__ exits,
                 const uint8_t* __restrict__ masked, const float* __restrict__ mask_prob,
                 const float* __restrict__ ce, const float* __restrict__ ar_ce,
                 const int32_t* __restrict__ ar_target, const int64_t* __restrict__ bounds,
                 int64_t S, int64_t rows, int K, float prior_c, float beta_mi, float beta_marg,
                 float* __restrict__ out, float* __restrict__ dgate, float* __restrict__ dce,
                 float dgate_scale, float* __restrict__ ws, const int32_t* __restrict__ nonfinite) {
  __shared__ float scratch[16];
  __shared__ float qbar_log[OBJ_MAX_DEPTH], prior_log[OBJ_MAX_DEPTH];
  __shared__ float sh_M, sh_wsum;
  float* logq = ws;               // [rows]
  float* credit = ws + rows;      // [rows]
  float* seg_R = ws + 2 * rows;   // [S]
  float* seg_Q = seg_R + S;       // [S]

  // ---- pass 1: counts, weight sum, exit-mass sums, nonfinite gates -----------
  float cnt = 0.f, wsum = 0.f, zsum = 0.f, h0 = 0.f, bad = 0.f;
  float qsum[OBJ_MAX_DEPTH];
  for (int d = 0; d < K; ++d) qsum[d] = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += OBJ_THREADS) {
    for (int d = 0; d < K; ++d)
      if (!isfinite(gates[(int64_t)d * rows + r])) bad = 1.f;
    if (!masked[r]) continue;
    if (exits[r] < 1 || exits[r] > K) { bad = 1.f; continue; }
    float le[OBJ_MAX_DEPTH];
    stick_logs(gates, rows, r, K, le);
    for (int d = 0; d < K; ++d) qsum[d] += expf(le[d]);
    cnt += 1.f;
    wsum += 1.0f / (mask_prob[r] + 1e-8f);
    zsum += (float)exits[r];
    h0 += sigmoidf_ref(gates[r]);
  }
  const float M = block_sum(cnt, scratch);
  const float W = block_sum(wsum, scratch);
  const float Z = block_sum(zsum, scratch);
  const float H0 = block_sum(h0, scratch);
  const float BAD = block_sum(bad, scratch);
  for (int d = 0; d < K; ++d) {
    const float q = block_sum(qsum[d], scratch);
    if (threadIdx.x == 0) qbar_log[d] = logf(fmaxf(M > 0.f ? q / M : 0.f, 1e-12f));
  }
  if (threadIdx.x == 0) {
    // log_softmax(-c * [1..K])
    float mx = -INFINITY;
    for (int d = 0; d < K; ++d) mx = fmaxf(mx, -prior_c * (float)(d + 1));
    float s = 0.f;
    for (int d = 0; d < K; ++d) s += expf(-prior_c * (float)(d + 1) - mx);
    for (int d = 0; d < K; ++d) prior_log[d] = -prior_c * (float)(d + 1) - mx - logf(s);
    sh_M = M;
    sh_wsum = W;
  }
  __syncthreads();

  // ---- pass 2: logq, credit, denoising, prediction and regularisation -------
  float den = 0.f, pred_sum = 0.f, reg_sum = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += OBJ_THREADS) {
    if (!masked[r] || exits[r] < 1 || exits[r] > K) {
      logq[r] = 0.f;
      credit[r] = 0.f;
      if (dce)
        for (int d = 0; d < K; ++d) dce[(int64_t)d * rows + r] = 0.f;
      continue;
    }
    float le[OBJ_MAX_DEPTH];
    stick_logs(gates, rows, r, K, le);
    const int z = exits[r];
    const float lq = le[z - 1];
    const float pred = ce[(int64_t)(z - 1) * rows + r] - ce[r];
    const float mi = beta_mi * (lq - qbar_log[z - 1]);
    const float budget = beta_marg * (qbar_log[z - 1] - prior_log[z - 1]);
    logq[r] = lq;
    credit[r] = (pred + mi) + budget;
    pred_sum += pred;
    reg_sum += mi + budget;
    const float w = (1.0f / (mask_prob[r] + 1e-8f)) / sh_wsum;
    float log_surv = 0.f, acc = 0.f;
    for (int d = 0; d < z; ++d) {
      const float stick = (d == z - 1) ? expf(log_surv) : expf(le[d]);
      acc += stick * ce[(int64_t)d * rows + r];
      log_surv -= softplusf(gates[(int64_t)d * rows + r]);
      // d denoising / d ce[d, r]: the detached stick times the row's weight
      if (dce) dce[(int64_t)d * rows + r] = w * stick;
    }
    if (dce)
      for (int d = z; d < K; ++d) dce[(int64_t)d * rows + r] = 0.f;
    den += w * acc;
  }
  const float DEN = block_sum(den, scratch);
  const float PRED = block_sum(pred_sum, scratch);
  const float REG = block_sum(reg_sum, scratch);

  // ---- autoregressive mean over depths (loss.py:12-32; model.py:183-184) ----
  float ar_sum = 0.f, ar_cnt = 0.f;
  for (int64_t r = threadIdx.x; ar_target != nullptr && r < rows; r += OBJ_THREADS) {
    if (ar_target[r] < 0) continue;
    ar_cnt += 1.f;
    for (int d = 0; d < K; ++d) ar_sum += ar_ce[(int64_t)d * rows + r];
  }
  const float AR_SUM = block_sum(ar_sum, scratch);
  const float AR_CNT = block_sum(ar_cnt, scratch);
  __syncthreads();  // logq / credit of every row are written

  // ---- segment sums: one wavefront per segment, rows in order ---------------
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int64_t s = wave; s < S; s += OBJ_THREADS / 64) {
    float R = 0.f, Q = 0.f;
    for (int64_t r = bounds[s] + lane; r < bounds[s + 1]; r += 64) {
      if (masked[r]) { R += credit[r]; Q += logq[r]; }
    }
    R = wave_sum(R);
    Q = wave_sum(Q);
    if (lane == 0) { seg_R[s] = R; seg_Q[s] = Q; }
  }
  __syncthreads();
  float act = 0.f;
  for (int64_t s = threadIdx.x; s < S; s += OBJ_THREADS) act += seg_R[s] * seg_Q[s];
  const float ACT_SUM = block_sum(act, scratch);

  // ---- d total / d gate (the actor's score function; loss.py:64-68, credit.py:38-40)
  for (int64_t r = threadIdx.x; r < rows; r += OBJ_THREADS) {
    if (!masked[r] || sh_M == 0.f || exits[r] < 1 || exits[r] > K) {
      for (int d = 0; d < K; ++d) dgate[(int64_t)d * rows + r] = 0.f;
      continue;
    }
    // segment of row r: bounds is sorted, S is small
    int64_t lo = 0, hi = S;
    while (hi - lo > 1) {
      int64_t mid = (lo + hi) >> 1;
      if (bounds[mid] <= r) lo = mid; else hi = mid;
    }
    const float a = dgate_scale * seg_R[lo] / sh_M;
    const int z = exits[r];
    for (int d = 0; d < K; ++d) {
      const float g = gates[(int64_t)d * rows + r];
      float dl = 0.f;
      if (d < z - 1) dl = -sigmoidf_ref(g);
      else if (d == z - 1 && z < K) dl = sigmoidf_ref(-g);
      dgate[(int64_t)d * rows + r] = a * dl;
    }
  }

  if (threadIdx.x == 0) {
    const float ar = AR_CNT > 0.f ? AR_SUM / (AR_CNT * (float)K) : 0.f;
    float den_v = 0.f, act_v = 0.f, zmean = 0.f, pmean = 0.f, rmean = 0.f, prof = 0.f, h0m = 0.f;
    if (M > 0.f) {
      den_v = DEN;
      act_v = ACT_SUM / M;
      zmean = Z / M;
      pmean = PRED / M;
      rmean = REG / M;
      for (int d = 0; d < K; ++d) prof += expf(qbar_log[d]) * (float)(d + 1);
      h0m = H0 / M;
    }
    float total = ((den_v + act_v) + ar) / 2.f;
    // 0 * sum(logits + gates) (model.py:186): a non-finite gate, or a
    // non-finite LM-head weight (whose logits column is then non-finite in
    // every row), makes the loss NaN; a non-finite readout row makes its gate
    // logit non-finite
    if (BAD > 0.f || (nonfinite != nullptr && *nonfinite != 0)) total = NAN;
    out[0] = total;
    out[1] = den_v;
    out[2] = act_v;
    out[3] = zmean;
    out[4] = pmean;
    out[5] = rmean;
    out[6] = prof;
    out[7] = h0m;
    out[8] = ar;
    out[9] = M;
  }
}

extern "C" int64_t alodlm_objective_workspace(int64_t rows, int64_t n_segments, int64_t max_depth) {
  (void)max_depth;
  return 2 * rows + 2 * n_segments;
}

extern "C" int alodlm_objective(const float* gates, const int32_t* exits, const uint8_t* masked,
                                const float* mask_prob, const float* ce_full, const float* ar_ce,
                                const int32_t* ar_target, const int64_t* bounds,
                                int64_t n_segments, int64_t rows, int64_t max_depth,
                                float depth_prior_c, float kl_beta_mi, float kl_beta_marg,
                                const int32_t* nonfinite, float* out, float* dgate,
                                float* workspace, void* stream) {
  ALODLM_CHECK_ARG(max_depth >= 2 && max_depth <= OBJ_MAX_DEPTH,
                   "objective: max_depth must be in [2, %d]", OBJ_MAX_DEPTH);
  ALODLM_CHECK_ARG(rows > 0 && n_segments > 0, "objective: empty input");
  objective_kernel<<<1, OBJ_THREADS, 0, as_stream(stream)>>>(
      gates, exits, masked, mask_prob, ce_full, ar_ce, ar_target, bounds, n_segments, rows,
      (int)max_depth, depth_prior_c, kl_beta_mi, kl_beta_marg, out, dgate, nullptr, 0.5f,
      workspace, nonfinite);
  ALODLM_CHECK_LAUNCH("objective");
  return ALODLM_OK;
}

extern "C" int alodlm_outcome_loss(const float* gates, const int32_t* exits, const uint8_t* masked,
                                   const float* mask_prob, const float* ce_full,
                                   const int64_t* bounds, int64_t n_segments, int64_t rows,
                                   int64_t max_depth, float depth_prior_c, float kl_beta_mi,
                                   float kl_beta_marg, float* out, float* dgate, float* dce,
                                   float* workspace, void* stream) {
  ALODLM_CHECK_ARG(max_depth >= 2 && max_depth <= OBJ_MAX_DEPTH,
                   "outcome_loss: max_depth must be in [2, %d]", OBJ_MAX_DEPTH);
  ALODLM_CHECK_ARG(rows > 0 && n_segments > 0, "outcome_loss: empty input");
  objective_kernel<<<1, OBJ_THREADS, 0, as_stream(stream)>>>(
      gates, exits, masked, mask_prob, ce_full, nullptr, nullptr, bounds, n_segments, rows,
      (int)max_depth, depth_prior_c, kl_beta_mi, kl_beta_marg, out, dgate, dce, 1.0f, workspace,
      nullptr);
  ALODLM_CHECK_LAUNCH("outcome_loss");
  return ALODLM_OK;
}

// ---------------------------------------------------------------------------
// Sequence credit primitives (alodlm/credit.py:7-40), one workgroup each.
// ---------------------------------------------------------------------------

// out[j] = segment of the j-th masked row (rows in order); *count = M.  The
// segment of row r is the number of segment ends bounds[1..S] at or before r
// (torch.bucketize(r, bounds[1:], right=True)).
__global__ void __launch_bounds__(1024)
masked_sequence_ids_kernel(const uint8_t* __restrict__ masked, const int64_t* __restrict__ bounds,
                           int64_t S, int64_t rows, int64_t* __restrict__ out,
                           int64_t* __restrict__ count) {
  __shared__ int64_t wave_total[16];
  __shared__ int64_t base;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x == 0) base = 0;
  __syncthreads();
  for (int64_t r0 = 0; r0 < rows; r0 += 1024) {
    const int64_t r = r0 + threadIdx.x;
    const bool m = r < rows && masked[r];
    const uint64_t ballot = __ballot(m);
    const int64_t before = __popcll(ballot & ((1ull << lane) - 1ull));
    if (lane == 0) wave_total[wave] = __popcll(ballot);
    __syncthreads();
    int64_t offset = base;
    for (int w = 0; w < wave; ++w) offset += wave_total[w];
    if (m) {
      int64_t lo = 0, hi = S;  // first s with bounds[s + 1] > r
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (bounds[mid + 1] <= r) lo = mid + 1; else hi = mid;
      }
      out[offset + before] = lo;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int64_t t = 0;
      for (int w = 0; w < 16; ++w) t += wave_total[w];
      base += t;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) count[0] = base;
}

extern "C" int alodlm_masked_sequence_ids(const uint8_t* masked, const int64_t* bounds,
                                          int64_t n_segments, int64_t rows, int64_t* out,
                                          int64_t* count, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && n_segments >= 1, "masked_sequence_ids: bad shape");
  masked_sequence_ids_kernel<<<1, 1024, 0, as_stream(stream)>>>(masked, bounds, n_segments, rows,
                                                               out, count);
  ALODLM_CHECK_LAUNCH("masked_sequence_ids");
  return ALODLM_OK;
}

// value[0] = sum_s R_s * Q_s / n with R_s = sum_{ids = s} credit and
// Q_s = sum_{ids = s} logq (rows in order within a segment; one wavefront
// per segment, fixed reduction order); dlogq[i] = R_{ids[i]} / n.
// `ws` holds 2 * S floats.
__global__ void __launch_bounds__(1024)
sequence_score_kernel(const float* __restrict__ credit, const float* __restrict__ logq,
                      const int64_t* __restrict__ ids, int64_t n, int64_t S,
                      float* __restrict__ value, float* __restrict__ dlogq,
                      float* __restrict__ ws) {
  __shared__ float scratch[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* seg_R = ws;
  float* seg_Q = ws + S;
  for (int64_t s = wave; s < S; s += 16) {
    float R = 0.f, Q = 0.f;
    for (int64_t i = lane; i < n; i += 64)
      if (ids[i] == s) { R += credit[i]; Q += logq[i]; }
    R = wave_sum(R);
    Q = wave_sum(Q);
    if (lane == 0) { seg_R[s] = R; seg_Q[s] = Q; }
  }
  __syncthreads();
  float acc = 0.f;
  for (int64_t s = threadIdx.x; s < S; s += 1024) acc += seg_R[s] * seg_Q[s];
  const float total = block_sum(acc, scratch);
  for (int64_t i = threadIdx.x; i < n; i += 1024) dlogq[i] = seg_R[ids[i]] / (float)n;
  if (threadIdx.x == 0) value[0] = total / (float)n;
}

extern "C" int alodlm_sequence_score(const float* credit, const float* logq, const int64_t* ids,
                                     int64_t n, int64_t sequence_count, float* value,
                                     float* dlogq, float* workspace, void* stream) {
  ALODLM_CHECK_ARG(n > 0 && sequence_count >= 1, "sequence_score: bad shape");
  sequence_score_kernel<<<1, 1024, 0, as_stream(stream)>>>(credit, logq, ids, n, sequence_count,
                                                          value, dlogq, workspace);
  ALODLM_CHECK_LAUNCH("sequence_score");
  return ALODLM_OK;
}

// AR targets of alodlm/loss.py:12-32 over the dual-stream rows of a pack:
// for the segment with dual-stream rows [start, end) and L = (end - start)/2,
// clean row start + i (i < L - 1) predicts labels[start/2 + 1 + i]; every
// other row, and ignored labels (-100), get -1.
__global__ void ar_targets_kernel(const int64_t* __restrict__ labels,
                                  const int64_t* __restrict__ bounds, int64_t S, int64_t rows,
                                  int32_t* __restrict__ target) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  int64_t lo = 0, hi = S;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (bounds[mid + 1] <= r) lo = mid + 1; else hi = mid;
  }
  int32_t t = -1;
  if (lo < S) {
    const int64_t start = bounds[lo], L = (bounds[lo + 1] - start) / 2, i = r - start;
    if (L >= 2 && i < L - 1) {
      const int64_t label = labels[start / 2 + 1 + i];
      if (label != -100) t = (int32_t)label;
    }
  }
  target[r] = t;
}

extern "C" int alodlm_ar_targets(const int64_t* labels, const int64_t* bounds, int64_t n_segments,
                                 int64_t rows, int32_t* target, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && n_segments >= 1, "ar_targets: bad shape");
  if (rows == 0) return ALODLM_OK;
  ar_targets_kernel<<<ceil_div_u(rows, 256), 256, 0, as_stream(stream)>>>(labels, bounds,
                                                                         n_segments, rows, target);
  ALODLM_CHECK_LAUNCH("ar_targets");
  return ALODLM_OK;
}
