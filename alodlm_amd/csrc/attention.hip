// GQA attention under the dual-stream training mask (alodlm/batch.py:23-31).
//
// Segment s occupies dual-stream rows [base, base + 2L): the clean stream
// [base, base + L) is causal; a noisy row in block b (of size B) sees the
// clean keys of earlier blocks [base, base + b*B) and, causally, the noisy
// rows of its own block.  The kernels enumerate exactly those key ranges, so
// no masked pair and no cross-segment pair is ever visited.
//
// Reference kernels (any dtype, any head_dim): one wavefront per (query row,
// head) in the forward and dQ passes and one per (key row, kv head) in the
// dK/dV pass; the wavefront spreads head_dim over its lanes.
#include <initializer_list>

#include "common.h"

#define ATT_MAX_PER_LANE 4  // head_dim <= 256

struct SegRow {
  int64_t base, L, i;  // segment start row, segment length, in-segment index (0..2L)
};

__device__ __forceinline__ SegRow seg_row(const int64_t* bounds, const int32_t* row_segment,
                                          int64_t r) {
  const int32_t s = row_segment[r];
  SegRow o;
  o.base = bounds[s];
  o.L = (bounds[s + 1] - o.base) / 2;
  o.i = r - o.base;
  return o;
}

// Key ranges [k0a, k1a) and [k0b, k1b) (absolute rows) seen by query row r.
__device__ __forceinline__ void query_key_ranges(const SegRow& q, int64_t B, int64_t& k0a,
                                                 int64_t& k1a, int64_t& k0b, int64_t& k1b) {
  if (q.i < q.L) {  // clean: causal over the clean stream
    k0a = q.base; k1a = q.base + q.i + 1;
    k0b = k1b = 0;
  } else {
    const int64_t j = q.i - q.L, blk = j / B;
    const int64_t clean_end = blk * B < q.L ? blk * B : q.L;
    k0a = q.base; k1a = q.base + clean_end;
    k0b = q.base + q.L + blk * B; k1b = q.base + q.i + 1;
  }
}

// Query ranges [q0a, q1a) and [q0b, q1b) (absolute rows) that see key row r.
__device__ __forceinline__ void key_query_ranges(const SegRow& k, int64_t B, int64_t& q0a,
                                                 int64_t& q1a, int64_t& q0b, int64_t& q1b) {
  if (k.i < k.L) {
    const int64_t blk = k.i / B;
    q0a = k.base + k.i; q1a = k.base + k.L;                  // later clean rows
    const int64_t first = (blk + 1) * B;                      // noisy rows of later blocks
    q0b = k.base + k.L + (first < k.L ? first : k.L); q1b = k.base + 2 * k.L;
  } else {
    const int64_t j = k.i - k.L, blk = j / B;
    const int64_t end = (blk + 1) * B < k.L ? (blk + 1) * B : k.L;
    q0a = k.base + k.i; q1a = k.base + k.L + end;             // same noisy block, causal
    q0b = q1b = 0;
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
attn_fwd_ref_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                    int64_t ldv, const int64_t* __restrict__ bounds,
                    const int32_t* __restrict__ row_segment, T* __restrict__ o,
                    float* __restrict__ lse, int64_t rows, int64_t nq, int64_t nkv, int64_t dh,
                    int64_t B, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= rows * nq) return;
  const int64_t r = item / nq, h = item % nq, hk = h / (nq / nkv);
  const int per = (int)((dh + 63) / 64);
  float qv[ATT_MAX_PER_LANE], acc[ATT_MAX_PER_LANE];
  for (int t = 0; t < per; ++t) {
    const int64_t e = lane + 64 * t;
    qv[t] = e < dh ? Elem<T>::load(q, (r * nq + h) * dh + e) : 0.f;
    acc[t] = 0.f;
  }
  const SegRow sr = seg_row(bounds, row_segment, r);
  int64_t ra[2][2];
  query_key_ranges(sr, B, ra[0][0], ra[0][1], ra[1][0], ra[1][1]);
  float m = -INFINITY, l = 0.f;
  for (int rg = 0; rg < 2; ++rg) {
    for (int64_t kr = ra[rg][0]; kr < ra[rg][1]; ++kr) {
      float s = 0.f;
      for (int t = 0; t < per; ++t) {
        const int64_t e = lane + 64 * t;
        if (e < dh) s += qv[t] * Elem<T>::load(k, (kr * nkv + hk) * dh + e);
      }
      s = wave_sum(s) * scale;
      const float mn = fmaxf(m, s);
      const float corr = expf(m - mn), p = expf(s - mn);
      l = l * corr + p;
      for (int t = 0; t < per; ++t) {
        const int64_t e = lane + 64 * t;
        const float vv = e < dh ? Elem<T>::load(v, kr * ldv + hk * dh + e) : 0.f;
        acc[t] = acc[t] * corr + p * vv;
      }
      m = mn;
    }
  }
  const float inv = 1.0f / l;
  for (int t = 0; t < per; ++t) {
    const int64_t e = lane + 64 * t;
    if (e < dh) Elem<T>::store(o, (r * nq + h) * dh + e, acc[t] * inv);
  }
  if (lane == 0) lse[h * rows + r] = m + logf(l);
}

// delta[h, r] = sum_e dO[r, h, e] * O[r, h, e]
template <typename T>
__global__ void __launch_bounds__(256)
attn_delta_kernel(const T* __restrict__ o, const T* __restrict__ dout, float* __restrict__ delta,
                  int64_t rows, int64_t nq, int64_t dh) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= rows * nq) return;
  const int64_t r = item / nq, h = item % nq;
  float s = 0.f;
  for (int64_t e = lane; e < dh; e += 64)
    s += Elem<T>::load(o, (r * nq + h) * dh + e) * Elem<T>::load(dout, (r * nq + h) * dh + e);
  s = wave_sum(s);
  if (lane == 0) delta[h * rows + r] = s;
}

template <typename T>
__global__ void __launch_bounds__(256)
attn_dq_ref_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                   int64_t ldv, const float* __restrict__ lse, const float* __restrict__ delta,
                   const T* __restrict__ dout, const int64_t* __restrict__ bounds,
                   const int32_t* __restrict__ row_segment, T* __restrict__ dq, int64_t rows,
                   int64_t nq, int64_t nkv, int64_t dh, int64_t B, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= rows * nq) return;
  const int64_t r = item / nq, h = item % nq, hk = h / (nq / nkv);
  const int per = (int)((dh + 63) / 64);
  float qv[ATT_MAX_PER_LANE], dov[ATT_MAX_PER_LANE], acc[ATT_MAX_PER_LANE];
  for (int t = 0; t < per; ++t) {
    const int64_t e = lane + 64 * t;
    qv[t] = e < dh ? Elem<T>::load(q, (r * nq + h) * dh + e) : 0.f;
    dov[t] = e < dh ? Elem<T>::load(dout, (r * nq + h) * dh + e) : 0.f;
    acc[t] = 0.f;
  }
  const float L_ = lse[h * rows + r], D = delta[h * rows + r];
  const SegRow sr = seg_row(bounds, row_segment, r);
  int64_t ra[2][2];
  query_key_ranges(sr, B, ra[0][0], ra[0][1], ra[1][0], ra[1][1]);
  for (int rg = 0; rg < 2; ++rg) {
    for (int64_t kr = ra[rg][0]; kr < ra[rg][1]; ++kr) {
      float s = 0.f, dp = 0.f;
      for (int t = 0; t < per; ++t) {
        const int64_t e = lane + 64 * t;
        if (e < dh) {
          s += qv[t] * Elem<T>::load(k, (kr * nkv + hk) * dh + e);
          dp += dov[t] * Elem<T>::load(v, kr * ldv + hk * dh + e);
        }
      }
      s = wave_sum(s) * scale;
      dp = wave_sum(dp);
      const float p = expf(s - L_);
      const float ds = p * (dp - D) * scale;
      for (int t = 0; t < per; ++t) {
        const int64_t e = lane + 64 * t;
        if (e < dh) acc[t] += ds * Elem<T>::load(k, (kr * nkv + hk) * dh + e);
      }
    }
  }
  for (int t = 0; t < per; ++t) {
    const int64_t e = lane + 64 * t;
    if (e < dh) Elem<T>::store(dq, (r * nq + h) * dh + e, acc[t]);
  }
}

template <typename T>
__global__ void __launch_bounds__(256)
attn_dkdv_ref_kernel(const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
                     int64_t ldv, const float* __restrict__ lse, const float* __restrict__ delta,
                     const T* __restrict__ dout, const int64_t* __restrict__ bounds,
                     const int32_t* __restrict__ row_segment, T* __restrict__ dk,
                     T* __restrict__ dv, int64_t lddv, int64_t rows, int64_t nq, int64_t nkv,
                     int64_t dh, int64_t B, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= rows * nkv) return;
  const int64_t r = item / nkv, hk = item % nkv;
  const int64_t group = nq / nkv;
  const int per = (int)((dh + 63) / 64);
  float kv[ATT_MAX_PER_LANE], vv[ATT_MAX_PER_LANE], dka[ATT_MAX_PER_LANE], dva[ATT_MAX_PER_LANE];
  for (int t = 0; t < per; ++t) {
    const int64_t e = lane + 64 * t;
    kv[t] = e < dh ? Elem<T>::load(k, (r * nkv + hk) * dh + e) : 0.f;
    vv[t] = e < dh ? Elem<T>::load(v, r * ldv + hk * dh + e) : 0.f;
    dka[t] = dva[t] = 0.f;
  }
  const SegRow sr = seg_row(bounds, row_segment, r);
  int64_t ra[2][2];
  key_query_ranges(sr, B, ra[0][0], ra[0][1], ra[1][0], ra[1][1]);
  for (int64_t h = hk * group; h < (hk + 1) * group; ++h) {
    for (int rg = 0; rg < 2; ++rg) {
      for (int64_t qr = ra[rg][0]; qr < ra[rg][1]; ++qr) {
        float s = 0.f, dp = 0.f;
        for (int t = 0; t < per; ++t) {
          const int64_t e = lane + 64 * t;
          if (e < dh) {
            s += kv[t] * Elem<T>::load(q, (qr * nq + h) * dh + e);
            dp += vv[t] * Elem<T>::load(dout, (qr * nq + h) * dh + e);
          }
        }
        s = wave_sum(s) * scale;
        dp = wave_sum(dp);
        const float p = expf(s - lse[h * rows + qr]);
        const float ds = p * (dp - delta[h * rows + qr]) * scale;
        for (int t = 0; t < per; ++t) {
          const int64_t e = lane + 64 * t;
          if (e < dh) {
            dva[t] += p * Elem<T>::load(dout, (qr * nq + h) * dh + e);
            dka[t] += ds * Elem<T>::load(q, (qr * nq + h) * dh + e);
          }
        }
      }
    }
  }
  for (int t = 0; t < per; ++t) {
    const int64_t e = lane + 64 * t;
    if (e < dh) {
      Elem<T>::store(dk, (r * nkv + hk) * dh + e, dka[t]);
      Elem<T>::store(dv, r * lddv + hk * dh + e, dva[t]);
    }
  }
}

static int check_attn(int64_t rows, int64_t nq, int64_t nkv, int64_t dh, int64_t B) {
  ALODLM_CHECK_ARG(rows >= 0 && nq > 0 && nkv > 0 && nq % nkv == 0, "attention: bad head counts");
  ALODLM_CHECK_ARG(dh > 0 && dh <= 64 * ATT_MAX_PER_LANE, "attention: head_dim must be <= 256");
  ALODLM_CHECK_ARG(B >= 1, "attention: block_size must be positive");
  return ALODLM_OK;
}

int fa_fwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                  const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* o,
                  float* lse, int64_t N, int nq, int nkv, int dh, int B, float scale,
                  hipStream_t st);
int fa_bwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                  const float* lse, const float* delta, const bf16_t* dout,
                  const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* dq,
                  bf16_t* dk, bf16_t* dv, int64_t lddv, int64_t N, int nq, int nkv, int dh,
                  int B, float scale, hipStream_t st);

int fa128_fwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                     const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* o,
                     float* lse, int64_t N, int nq, int nkv, int B, float scale, hipStream_t st);
int fa128_bwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                     const float* lse, const bf16_t* o, float* delta, const bf16_t* dout,
                     const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* dq,
                     bf16_t* dk, bf16_t* dv, int64_t lddv, int64_t N, int nq, int nkv, int B,
                     float scale, const int64_t* ds_base, int64_t ds_blocks, hipStream_t st);

// The MFMA kernels take bf16, head_dim 64 or 128, 16-byte aligned rows and a
// tile table; everything else runs the reference kernels above.
static bool use_mfma(int dtype, int64_t dh, const int32_t* tiles, int64_t ldv,
                     std::initializer_list<const void*> ptrs) {
  if (dtype != ALODLM_BF16 || tiles == nullptr || (dh != 64 && dh != 128) || ldv % 8) return false;
  for (const void* p : ptrs)
    if (reinterpret_cast<uintptr_t>(p) % 16) return false;
  return true;
}

extern "C" int alodlm_attention_fwd(const void* q, const void* k, const void* v, int64_t ldv,
                                    const int64_t* bounds, const int32_t* row_segment,
                                    const int32_t* tiles, int64_t n_tiles, void* o, float* lse,
                                    int64_t rows, int64_t nq, int64_t nkv, int64_t dh,
                                    int64_t block_size, int dtype, void* stream) {
  int rc = check_attn(rows, nq, nkv, dh, block_size);
  if (rc) return rc;
  if (rows == 0) return ALODLM_OK;
  const float scale = 1.0f / sqrtf((float)dh);
  if (use_mfma(dtype, dh, tiles, ldv, {q, k, v, o})) {
    if (n_tiles == 0) return ALODLM_OK;
    ALODLM_CHECK_ARG(n_tiles <= 65535, "attention: too many 128-row tiles (%lld)", (long long)n_tiles);
    if (dh == 128)
      return fa128_fwd_launch((const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ldv, bounds,
                              tiles, n_tiles, (bf16_t*)o, lse, rows, (int)nq, (int)nkv,
                              (int)block_size, scale, as_stream(stream));
    return fa_fwd_launch((const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ldv, bounds, tiles,
                         n_tiles, (bf16_t*)o, lse, rows, (int)nq, (int)nkv, (int)dh,
                         (int)block_size, scale, as_stream(stream));
  }
  ALODLM_DISPATCH(dtype, T, {
    attn_fwd_ref_kernel<T><<<ceil_div_u(rows * nq, 4), 256, 0, as_stream(stream)>>>(
        (const T*)q, (const T*)k, (const T*)v, ldv, bounds, row_segment, (T*)o, lse, rows, nq,
        nkv, dh, block_size, scale);
  });
  ALODLM_CHECK_LAUNCH("attention_fwd");
  return ALODLM_OK;
}

int64_t fa128_bwd_workspace(int64_t N, int nq, int nkv, int64_t n_tiles, int64_t ds_blocks);

// 32x32 dS blocks per query head that the mask allows in a pack (the stored-dS
// backward's buffer): per segment of L tokens, T (T + 1) with T = ceil(L / 32);
// 0 unless block_size is 32.  base_out (S + 1 entries, may be NULL) receives
// each segment's first block and the total.  Host only.
extern "C" int64_t alodlm_attention_ds_blocks(const int64_t* token_offsets, int64_t segments,
                                              int64_t block_size, int64_t* base_out) {
  if (token_offsets == nullptr || segments < 0) return 0;
  int64_t total = 0;
  for (int64_t s = 0; s < segments; ++s) {
    if (base_out) base_out[s] = total;
    const int64_t L = token_offsets[s + 1] - token_offsets[s];
    const int64_t T = (L + 31) / 32;
    total += T * (T + 1);
  }
  if (base_out) base_out[segments] = total;
  return block_size == 32 ? total : 0;
}

extern "C" int64_t alodlm_attention_bwd_workspace(int64_t rows, int64_t nq, int64_t nkv,
                                                  int64_t dh, int64_t n_tiles, int64_t ds_blocks) {
  // delta [nq][rows]; the head_dim-128 kernels may also keep dK/dV partials
  // and the stored dS blocks
  if (dh == 128 && nq > 0 && nkv > 0)
    return fa128_bwd_workspace(rows, (int)nq, (int)nkv, n_tiles, ds_blocks);
  return rows * nq;
}

extern "C" int alodlm_attention_bwd(const void* q, const void* k, const void* v, int64_t ldv,
                                    const void* o, const float* lse, const void* dout,
                                    const int64_t* bounds, const int32_t* row_segment,
                                    const int32_t* tiles, int64_t n_tiles, void* dq, void* dk,
                                    void* dv, int64_t lddv, float* workspace,
                                    const int64_t* ds_base, int64_t ds_blocks, int64_t rows,
                                    int64_t nq, int64_t nkv, int64_t dh, int64_t block_size,
                                    int dtype, void* stream) {
  int rc = check_attn(rows, nq, nkv, dh, block_size);
  if (rc) return rc;
  if (rows == 0) return ALODLM_OK;
  const float scale = 1.0f / sqrtf((float)dh);
  hipStream_t st = as_stream(stream);
  float* delta = workspace;
  const bool mfma = use_mfma(dtype, dh, tiles, ldv, {q, k, v, o, dout, dq, dk, dv}) && lddv % 8 == 0;
  if (mfma && dh == 128) {
    // the head_dim-128 kernels compute delta themselves
    if (n_tiles == 0) return ALODLM_OK;
    ALODLM_CHECK_ARG(n_tiles <= 65535, "attention: too many 128-row tiles (%lld)", (long long)n_tiles);
    return fa128_bwd_launch((const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ldv, lse,
                            (const bf16_t*)o, delta, (const bf16_t*)dout, bounds, tiles, n_tiles,
                            (bf16_t*)dq, (bf16_t*)dk, (bf16_t*)dv, lddv, rows, (int)nq, (int)nkv,
                            (int)block_size, scale, ds_base, ds_blocks, st);
  }
  ALODLM_DISPATCH(dtype, T, {
    attn_delta_kernel<T><<<ceil_div_u(rows * nq, 4), 256, 0, st>>>((const T*)o, (const T*)dout,
                                                                   delta, rows, nq, dh);
  });
  ALODLM_CHECK_LAUNCH("attention_delta");
  if (mfma) {  // head_dim 64
    if (n_tiles == 0) return ALODLM_OK;
    ALODLM_CHECK_ARG(n_tiles <= 65535, "attention: too many 128-row tiles (%lld)", (long long)n_tiles);
    return fa_bwd_launch((const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ldv, lse, delta,
                         (const bf16_t*)dout, bounds, tiles, n_tiles, (bf16_t*)dq, (bf16_t*)dk,
                         (bf16_t*)dv, lddv, rows, (int)nq, (int)nkv, (int)dh, (int)block_size,
                         scale, st);
  }
  ALODLM_DISPATCH(dtype, T, {
    attn_dq_ref_kernel<T><<<ceil_div_u(rows * nq, 4), 256, 0, st>>>(
        (const T*)q, (const T*)k, (const T*)v, ldv, lse, delta, (const T*)dout, bounds,
        row_segment, (T*)dq, rows, nq, nkv, dh, block_size, scale);
    attn_dkdv_ref_kernel<T><<<ceil_div_u(rows * nkv, 4), 256, 0, st>>>(
        (const T*)q, (const T*)k, (const T*)v, ldv, lse, delta, (const T*)dout, bounds,
        row_segment, (T*)dk, (T*)dv, lddv, rows, nq, nkv, dh, block_size, scale);
  });
  ALODLM_CHECK_LAUNCH("attention_bwd");
  return ALODLM_OK;
}
