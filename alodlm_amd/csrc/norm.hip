// RMSNorm family: layer norms, q/k head norms fused with rotary, the final
// norm fused with the gate head, and the carry norm fused with re-embedding.
//
// One wavefront owns one row (or one head of one row); sums are wavefront
// reductions.  Row access is 16-byte vectorised when the width is a multiple
// of 8 (always true for Qwen3 shapes), otherwise scalar.
#include "common.h"

#define NORM_WAVES 4

// Iterate the columns a lane owns: 8-wide chunks when V8, else single elements.
#define FOR_LANE_CHUNKS(V8, cols, lane, c)                                   \
  for (int64_t c = (V8) ? (int64_t)(lane) * 8 : (int64_t)(lane); c < (cols); \
       c += (V8) ? 512 : 64)

template <typename T, bool V8>
__device__ __forceinline__ void load_chunk(const T* p, int64_t c, float* v) {
  if (V8) Vec8<T>::load(p + c, v);
  else v[0] = Elem<T>::load(p, c);
}
template <typename T, bool V8>
__device__ __forceinline__ void store_chunk(T* p, int64_t c, const float* v) {
  if (V8) Vec8<T>::store(p + c, v);
  else Elem<T>::store(p, c, v[0]);
}

// ---------------------------------------------------------------------------
// y = w * cast(x * rsqrt(mean(x^2) + eps))   ([tf] modeling_qwen3.py:59-64)
// ---------------------------------------------------------------------------
template <typename T, bool V8>
__global__ void __launch_bounds__(64 * NORM_WAVES)
rmsnorm_fwd_kernel(const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
                   float* __restrict__ rstd, int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * NORM_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * cols;
  T* yr = y + row * cols;
  constexpr int W = V8 ? 8 : 1;
  float ss = 0.f;
  FOR_LANE_CHUNKS(V8, cols, lane, c) {
    float v[8];
    load_chunk<T, V8>(xr, c, v);
#pragma unroll
    for (int i = 0; i < W; ++i) ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)cols + eps);
  if (lane == 0 && rstd) rstd[row] = r;
  FOR_LANE_CHUNKS(V8, cols, lane, c) {
    float v[8], g[8];
    load_chunk<T, V8>(xr, c, v);
    load_chunk<T, V8>(w, c, g);
#pragma unroll
    for (int i = 0; i < W; ++i) v[i] = g[i] * Elem<T>::round(v[i] * r);
    store_chunk<T, V8>(yr, c, v);
  }
}

// dx = dres + r*(dy*w) - x*r^3*mean((dy*w)*x);  partial[blk, :] = sum dy*cast(x*r)
// Rows with skip_exits[row] <= skip_depth take dy = 0 (their output was
// replaced by a re-embedded token; alodlm/model.py:153-154): dx = dres.
template <typename T, bool V8>
__global__ void __launch_bounds__(64)
rmsnorm_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x, const float* __restrict__ rstd,
                   const T* __restrict__ w, const T* dres, T* dx, float* __restrict__ partial,
                   int64_t rows, int64_t cols, int64_t rows_per_block,
                   const int32_t* __restrict__ skip_exits, int64_t skip_depth) {
  extern __shared__ float dw_lds[];
  const int lane = threadIdx.x;
  constexpr int W = V8 ? 8 : 1;
  for (int64_t c = lane; c < cols; c += 64) dw_lds[c] = 0.f;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
  for (int64_t row = r0; row < r1; ++row) {
    const T* dyr = dy + row * cols;
    const T* xr = x + row * cols;
    const float r = rstd[row];
    if (skip_exits && skip_exits[row] <= skip_depth) {
      FOR_LANE_CHUNKS(V8, cols, lane, c) {
        float o[8];
        if (dres) load_chunk<T, V8>(dres + row * cols, c, o);
        else {
#pragma unroll
          for (int i = 0; i < W; ++i) o[i] = 0.f;
        }
        store_chunk<T, V8>(dx + row * cols, c, o);
      }
      continue;
    }
    float s = 0.f;
    FOR_LANE_CHUNKS(V8, cols, lane, c) {
      float a[8], b[8], g[8];
      load_chunk<T, V8>(dyr, c, a);
      load_chunk<T, V8>(xr, c, b);
      load_chunk<T, V8>(w, c, g);
#pragma unroll
      for (int i = 0; i < W; ++i) {
        s += a[i] * g[i] * b[i];
        dw_lds[c + i] += a[i] * Elem<T>::round(b[i] * r);
      }
    }
    s = wave_sum(s);
    const float k = s * r * r * r / (float)cols;
    FOR_LANE_CHUNKS(V8, cols, lane, c) {
      float a[8], b[8], g[8], o[8];
      load_chunk<T, V8>(dyr, c, a);
      load_chunk<T, V8>(xr, c, b);
      load_chunk<T, V8>(w, c, g);
      if (dres) load_chunk<T, V8>(dres + row * cols, c, o);
      else {
#pragma unroll
        for (int i = 0; i < W; ++i) o[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) o[i] += r * a[i] * g[i] - b[i] * k;
      store_chunk<T, V8>(dx + row * cols, c, o);
    }
  }
  for (int64_t c = lane; c < cols; c += 64) partial[(int64_t)blockIdx.x * cols + c] = dw_lds[c];
}

// out[c] += sum_p partial[p, c]  (fixed order)
__global__ void column_reduce_kernel(const float* __restrict__ partial, int64_t nparts,
                                     int64_t cols, float* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float s = 0.f;
  for (int64_t p = 0; p < nparts; ++p) s += partial[p * cols + c];
  out[c] += s;
}

// first[c] += sum_p partial[p, c] for c < half; second[c-half] for the rest.
__global__ void split_column_reduce_kernel(const float* __restrict__ partial, int64_t nparts,
                                           int64_t half, float* __restrict__ first,
                                           float* __restrict__ second) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= 2 * half) return;
  float s = 0.f;
  for (int64_t p = 0; p < nparts; ++p) s += partial[p * 2 * half + c];
  if (c < half) first[c] += s;
  else second[c - half] += s;
}

static const int64_t kNormBwdRows = 64;

extern "C" int alodlm_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd,
                                  int64_t rows, int64_t cols, float eps, int dtype, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && cols > 0, "rmsnorm_fwd: bad shape");
  if (rows == 0) return ALODLM_OK;
  const bool v8 = cols % 8 == 0 && aligned8(x, dtype) && aligned8(y, dtype) && aligned8(w, dtype);
  ALODLM_DISPATCH(dtype, T, {
    dim3 grid(ceil_div_u(rows, NORM_WAVES));
    if (v8) rmsnorm_fwd_kernel<T, true><<<grid, 64 * NORM_WAVES, 0, as_stream(stream)>>>(
        (const T*)x, (const T*)w, (T*)y, rstd, rows, cols, eps);
    else rmsnorm_fwd_kernel<T, false><<<grid, 64 * NORM_WAVES, 0, as_stream(stream)>>>(
        (const T*)x, (const T*)w, (T*)y, rstd, rows, cols, eps);
  });
  ALODLM_CHECK_LAUNCH("rmsnorm_fwd");
  return ALODLM_OK;
}

extern "C" int64_t alodlm_rmsnorm_bwd_workspace(int64_t rows, int64_t cols) {
  return ((rows + kNormBwdRows - 1) / kNormBwdRows) * cols;
}

static int rmsnorm_bwd_launch(const void* dy, const void* x, const float* rstd, const void* w,
                              const void* dres, void* dx, float* dw_accum, float* workspace,
                              int64_t rows, int64_t cols, int dtype, const int32_t* skip_exits,
                              int64_t skip_depth, hipStream_t st) {
  ALODLM_CHECK_ARG(rows >= 0 && cols > 0, "rmsnorm_bwd: bad shape");
  ALODLM_CHECK_ARG(cols * 4 <= 64 * 1024, "rmsnorm_bwd: cols too large");
  if (rows == 0) return ALODLM_OK;
  const bool v8 = cols % 8 == 0 && aligned8(x, dtype) && aligned8(dy, dtype) &&
                  aligned8(dx, dtype) && aligned8(w, dtype) && (!dres || aligned8(dres, dtype));
  const int64_t nparts = (rows + kNormBwdRows - 1) / kNormBwdRows;
  ALODLM_DISPATCH(dtype, T, {
    size_t lds = (size_t)cols * sizeof(float);
    if (v8) rmsnorm_bwd_kernel<T, true><<<(unsigned)nparts, 64, lds, st>>>(
        (const T*)dy, (const T*)x, rstd, (const T*)w, (const T*)dres, (T*)dx, workspace, rows,
        cols, kNormBwdRows, skip_exits, skip_depth);
    else rmsnorm_bwd_kernel<T, false><<<(unsigned)nparts, 64, lds, st>>>(
        (const T*)dy, (const T*)x, rstd, (const T*)w, (const T*)dres, (T*)dx, workspace, rows,
        cols, kNormBwdRows, skip_exits, skip_depth);
  });
  ALODLM_CHECK_LAUNCH("rmsnorm_bwd");
  if (dw_accum) {
    column_reduce_kernel<<<ceil_div_u(cols, 256), 256, 0, st>>>(workspace, nparts, cols, dw_accum);
    ALODLM_CHECK_LAUNCH("rmsnorm_bwd_reduce");
  }
  return ALODLM_OK;
}

extern "C" int alodlm_rmsnorm_bwd(const void* dy, const void* x, const float* rstd, const void* w,
                                  const void* dres, void* dx, float* dw_accum, float* workspace,
                                  int64_t rows, int64_t cols, int dtype, void* stream) {
  return rmsnorm_bwd_launch(dy, x, rstd, w, dres, dx, dw_accum, workspace, rows, cols, dtype,
                            nullptr, 0, as_stream(stream));
}

extern "C" int alodlm_carry_select_bwd(const void* dy, const void* x, const float* rstd,
                                       const void* wf, const int32_t* exits, int64_t depth,
                                       const int64_t* original, const void* dres, void* dx,
                                       float* dwf_accum, float* dtable, float* workspace,
                                       int64_t rows, int64_t hidden, int64_t vocab, int dtype,
                                       void* stream) {
  // re-embedded rows (exits <= depth) send their gradient to the embedding table
  int rc = alodlm_embed_scatter_add(dy, original, exits, depth, dtable, rows, hidden, vocab, dtype,
                                    stream);
  if (rc) return rc;
  // carried rows go back through the carry norm into the previous depth's core output
  return rmsnorm_bwd_launch(dy, x, rstd, wf, dres, dx, dwf_accum, workspace, rows, hidden, dtype,
                            exits, depth, as_stream(stream));
}

// ---------------------------------------------------------------------------
// q_norm / k_norm + rotary.  One wavefront per (row, head); a lane owns the
// rotary pairs (i, i + dh/2) for i = lane, lane + 64, ...  cos/sin are
// computed in float at the row's position and cast to the storage type like
// the reference's rotary table ([tf] :126-137); q*cos and rotate(q)*sin and
// their sum each round to the storage type (alodlm/model.py:41-46).
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(64 * NORM_WAVES)
qknorm_rope_fwd_kernel(const T* __restrict__ qkv, const T* __restrict__ wq, const T* __restrict__ wk,
                       const int64_t* __restrict__ positions, const float* __restrict__ inv_freq,
                       T* __restrict__ q_out, T* __restrict__ k_out, int64_t rows, int64_t nq,
                       int64_t nkv, int64_t dh, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * NORM_WAVES + (threadIdx.x >> 6);
  const int64_t heads = nq + nkv;
  if (item >= rows * heads) return;
  const int64_t row = item / heads, head = item % heads;
  const bool is_q = head < nq;
  const T* src = qkv + row * (nq + 2 * nkv) * dh + head * dh;
  const T* w = is_q ? wq : wk;
  T* dst = is_q ? q_out + (row * nq + head) * dh : k_out + (row * nkv + (head - nq)) * dh;
  const int64_t half = dh / 2;
  float ss = 0.f;
  for (int64_t i = lane; i < dh; i += 64) {
    float v = Elem<T>::load(src, i);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)dh + eps);
  const float pos = (float)positions[row];
  for (int64_t i = lane; i < half; i += 64) {
    const float a = Elem<T>::round(Elem<T>::load(w, i) * Elem<T>::round(Elem<T>::load(src, i) * r));
    const float b = Elem<T>::round(Elem<T>::load(w, i + half) *
                                   Elem<T>::round(Elem<T>::load(src, i + half) * r));
    const float ang = pos * inv_freq[i];
    const float c = Elem<T>::round(cosf(ang)), s = Elem<T>::round(sinf(ang));
    Elem<T>::store(dst, i, Elem<T>::round(a * c) + Elem<T>::round(-b * s));
    Elem<T>::store(dst, i + half, Elem<T>::round(b * c) + Elem<T>::round(a * s));
  }
}

// Backward of the above.  dt = rotary^T d(out); then the RMSNorm backward over
// dh.  partial[blk, 0:dh] / [blk, dh:2dh] collect the q/k norm-weight grads.
template <typename T>
__global__ void __launch_bounds__(64)
qknorm_rope_bwd_kernel(const T* __restrict__ dq, const T* __restrict__ dk, const T* __restrict__ qkv,
                       const T* __restrict__ wq, const T* __restrict__ wk,
                       const int64_t* __restrict__ positions, const float* __restrict__ inv_freq,
                       T* __restrict__ dqkv, float* __restrict__ partial, int64_t rows, int64_t nq,
                       int64_t nkv, int64_t dh, float eps, int64_t rows_per_block) {
  extern __shared__ float lds_w[];  // [2*dh]: q then k weight-grad partials
  const int lane = threadIdx.x;
  for (int64_t i = lane; i < 2 * dh; i += 64) lds_w[i] = 0.f;
  const int64_t half = dh / 2;
  const int64_t width = (nq + 2 * nkv) * dh;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
  for (int64_t row = r0; row < r1; ++row) {
    const float pos = (float)positions[row];
    for (int64_t head = 0; head < nq + nkv; ++head) {
      const bool is_q = head < nq;
      const T* src = qkv + row * width + head * dh;
      const T* w = is_q ? wq : wk;
      const T* g = is_q ? dq + (row * nq + head) * dh : dk + (row * nkv + (head - nq)) * dh;
      float* acc = lds_w + (is_q ? 0 : dh);
      float ss = 0.f;
      for (int64_t i = lane; i < dh; i += 64) {
        float v = Elem<T>::load(src, i);
        ss += v * v;
      }
      ss = wave_sum(ss);
      const float r = 1.0f / sqrtf(ss / (float)dh + eps);
      // dt (gradient wrt the normalised, weighted value) and sum(dt*w*x)
      float s = 0.f;
      for (int64_t i = lane; i < half; i += 64) {
        const float ang = pos * inv_freq[i];
        const float c = Elem<T>::round(cosf(ang)), sn = Elem<T>::round(sinf(ang));
        const float go = Elem<T>::load(g, i), gh = Elem<T>::load(g, i + half);
        const float dta = go * c + gh * sn;      // d/d t[i]
        const float dtb = gh * c - go * sn;      // d/d t[i+half]
        const float xa = Elem<T>::load(src, i), xb = Elem<T>::load(src, i + half);
        const float wa = Elem<T>::load(w, i), wb = Elem<T>::load(w, i + half);
        s += dta * wa * xa + dtb * wb * xb;
        acc[i] += dta * Elem<T>::round(xa * r);
        acc[i + half] += dtb * Elem<T>::round(xb * r);
      }
      s = wave_sum(s);
      const float k = s * r * r * r / (float)dh;
      T* out = dqkv + row * width + head * dh;
      for (int64_t i = lane; i < half; i += 64) {
        const float ang = pos * inv_freq[i];
        const float c = Elem<T>::round(cosf(ang)), sn = Elem<T>::round(sinf(ang));
        const float go = Elem<T>::load(g, i), gh = Elem<T>::load(g, i + half);
        const float dta = go * c + gh * sn;
        const float dtb = gh * c - go * sn;
        const float xa = Elem<T>::load(src, i), xb = Elem<T>::load(src, i + half);
        const float wa = Elem<T>::load(w, i), wb = Elem<T>::load(w, i + half);
        Elem<T>::store(out, i, r * dta * wa - xa * k);
        Elem<T>::store(out, i + half, r * dtb * wb - xb * k);
      }
    }
  }
  for (int64_t i = lane; i < 2 * dh; i += 64) partial[(int64_t)blockIdx.x * 2 * dh + i] = lds_w[i];
}

static const int64_t kQkBwdRows = 32;

extern "C" int alodlm_qknorm_rope_fwd(const void* qkv, const void* wq, const void* wk,
                                      const int64_t* positions, const float* inv_freq, void* q_out,
                                      void* k_out, int64_t rows, int64_t nq, int64_t nkv,
                                      int64_t dh, float eps, int dtype, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && nq > 0 && nkv > 0 && dh > 0 && dh % 2 == 0,
                   "qknorm_rope_fwd: bad shape");
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    qknorm_rope_fwd_kernel<T><<<ceil_div_u(rows * (nq + nkv), NORM_WAVES), 64 * NORM_WAVES, 0,
                                as_stream(stream)>>>(
        (const T*)qkv, (const T*)wq, (const T*)wk, positions, inv_freq, (T*)q_out, (T*)k_out,
        rows, nq, nkv, dh, eps);
  });
  ALODLM_CHECK_LAUNCH("qknorm_rope_fwd");
  return ALODLM_OK;
}

extern "C" int64_t alodlm_qknorm_rope_bwd_workspace(int64_t rows, int64_t nq, int64_t nkv,
                                                    int64_t dh) {
  (void)nq; (void)nkv;
  return ((rows + kQkBwdRows - 1) / kQkBwdRows) * 2 * dh;
}

extern "C" int alodlm_qknorm_rope_bwd(const void* dq, const void* dk, const void* qkv,
                                      const void* wq, const void* wk, const int64_t* positions,
                                      const float* inv_freq, void* dqkv, float* dwq_accum,
                                      float* dwk_accum, float* workspace, int64_t rows, int64_t nq,
                                      int64_t nkv, int64_t dh, float eps, int dtype, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && nq > 0 && nkv > 0 && dh > 0 && dh % 2 == 0,
                   "qknorm_rope_bwd: bad shape");
  if (rows == 0) return ALODLM_OK;
  const int64_t nparts = (rows + kQkBwdRows - 1) / kQkBwdRows;
  hipStream_t st = as_stream(stream);
  ALODLM_DISPATCH(dtype, T, {
    qknorm_rope_bwd_kernel<T><<<(unsigned)nparts, 64, 2 * dh * sizeof(float), st>>>(
        (const T*)dq, (const T*)dk, (const T*)qkv, (const T*)wq, (const T*)wk, positions,
        inv_freq, (T*)dqkv, workspace, rows, nq, nkv, dh, eps, kQkBwdRows);
  });
  ALODLM_CHECK_LAUNCH("qknorm_rope_bwd");
  // partial layout [nparts, 2*dh]: the q half goes to dwq, the k half to dwk
  split_column_reduce_kernel<<<ceil_div_u(2 * dh, 256), 256, 0, st>>>(workspace, nparts, dh,
                                                                      dwq_accum, dwk_accum);
  ALODLM_CHECK_LAUNCH("qknorm_rope_bwd_reduce");
  return ALODLM_OK;
}
