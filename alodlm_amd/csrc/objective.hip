// The step objective on [K, rows]: truncated-stick denoising, the sequence
// score-function actor with the geometric prior and the sampled-history
// marginal, the autoregressive mean, the metrics, and d(total)/d(gate).
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
                 float* __restrict__ out, float* __restrict__ dgate, float* __restrict__ ws) {
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
    if (!masked[r] || exits[r] < 1 || exits[r] > K) { logq[r] = 0.f; credit[r] = 0.f; continue; }
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
    }
    den += w * acc;
  }
  const float DEN = block_sum(den, scratch);
  const float PRED = block_sum(pred_sum, scratch);
  const float REG = block_sum(reg_sum, scratch);

  // ---- autoregressive mean over depths (loss.py:12-32; model.py:183-184) ----
  float ar_sum = 0.f, ar_cnt = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += OBJ_THREADS) {
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
    const float a = 0.5f * seg_R[lo] / sh_M;
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
    if (BAD > 0.f) total = NAN;  // 0 * sum(gates) propagates non-finite gates (model.py:186)
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
                                float* out, float* dgate, float* workspace, void* stream) {
  ALODLM_CHECK_ARG(max_depth >= 2 && max_depth <= OBJ_MAX_DEPTH,
                   "objective: max_depth must be in [2, %d]", OBJ_MAX_DEPTH);
  ALODLM_CHECK_ARG(rows > 0 && n_segments > 0, "objective: empty input");
  objective_kernel<<<1, OBJ_THREADS, 0, as_stream(stream)>>>(
      gates, exits, masked, mask_prob, ce_full, ar_ce, ar_target, bounds, n_segments, rows,
      (int)max_depth, depth_prior_c, kl_beta_mi, kl_beta_marg, out, dgate, workspace);
  ALODLM_CHECK_LAUNCH("objective");
  return ALODLM_OK;
}
