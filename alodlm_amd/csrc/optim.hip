// Gradient clipping and AdamW over a list of tensors
// (torch.nn.utils.clip_grad_norm_ and torch.optim.AdamW as called at
// alodlm/train.py:49,140,143).
//
// The tensor list is cut into fixed-size chunks on the host once; chunk c
// covers elements [chunk_start[c], chunk_start[c] + chunk_size) of tensor
// chunk_tensor[c].  Both kernels walk that table, so a 311M-element embedding
// and a 128-element norm weight are handled by the same launch.  AdamW keeps a
// float master copy, first and second moments per tensor (HBM traffic per
// element: grad + master r/w + m r/w + v r/w + param w).
#include "common.h"

#define OPT_THREADS 256

template <typename T>
__global__ void __launch_bounds__(OPT_THREADS)
grad_sumsq_kernel(const void* const* __restrict__ grads, const int32_t* __restrict__ chunk_tensor,
                  const int64_t* __restrict__ chunk_start, const int64_t* __restrict__ numels,
                  int64_t chunk_size, float* __restrict__ partial) {
  __shared__ float scratch[OPT_THREADS / 64];
  const int64_t c = blockIdx.x;
  const int32_t t = chunk_tensor[c];
  const T* g = reinterpret_cast<const T*>(grads[t]);
  const int64_t beg = chunk_start[c];
  const int64_t end = beg + chunk_size < numels[t] ? beg + chunk_size : numels[t];
  float s = 0.f;
  int64_t i = beg;
  if ((reinterpret_cast<uintptr_t>(g + beg) & 15) == 0) {
    // 16-byte pieces while whole ones remain (the test is uniform per block)
    const int64_t vec_end = beg + (end - beg) / (16 / sizeof(T)) * (16 / sizeof(T));
    if constexpr (sizeof(T) == 2) {
      for (int64_t j = beg + threadIdx.x * 8; j < vec_end; j += OPT_THREADS * 8) {
        float v[8];
        Vec8<T>::load(g + j, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[e] * v[e];
      }
    } else {
      for (int64_t j = beg + threadIdx.x * 4; j < vec_end; j += OPT_THREADS * 4) {
        const float4 v = *reinterpret_cast<const float4*>(g + j);
        s += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
    }
    i = vec_end;
  }
  for (i += threadIdx.x; i < end; i += OPT_THREADS) {
    const float v = Elem<T>::load(g, i);
    s += v * v;
  }
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) partial[c] = s;
}

__global__ void __launch_bounds__(1024)
final_norm_kernel(const float* __restrict__ partial, int64_t n, float* __restrict__ total) {
  __shared__ float scratch[16];
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += partial[i];
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) total[0] = sqrtf(s);
}

template <typename T, typename G>
__global__ void __launch_bounds__(OPT_THREADS)
adamw_kernel(void* const* __restrict__ params, float* const* __restrict__ master,
             float* const* __restrict__ exp_avg, float* const* __restrict__ exp_avg_sq,
             const void* const* __restrict__ grads, const int32_t* __restrict__ chunk_tensor,
             const int64_t* __restrict__ chunk_start, const int64_t* __restrict__ numels,
             const float* __restrict__ weight_decay, int64_t chunk_size,
             const float* __restrict__ total_norm, float max_norm, float lr, float beta1,
             float beta2, float eps, float step_size, float bc2_sqrt) {
  const int64_t c = blockIdx.x;
  const int32_t t = chunk_tensor[c];
  const int64_t beg = chunk_start[c];
  const int64_t end = beg + chunk_size < numels[t] ? beg + chunk_size : numels[t];
  float clip = 1.0f;
  if (total_norm) clip = fminf(1.0f, max_norm / (total_norm[0] + 1e-6f));
  const float decay = 1.0f - lr * weight_decay[t];
  // the tables hold generic pointers to device memory: the casts let every
  // access be a global (not flat) memory instruction
#define OPT_GLOBAL __attribute__((address_space(1)))
  OPT_GLOBAL T* p = (OPT_GLOBAL T*)reinterpret_cast<T*>(params[t]);
  OPT_GLOBAL float* w = (OPT_GLOBAL float*)master[t];
  OPT_GLOBAL float* m = (OPT_GLOBAL float*)exp_avg[t];
  OPT_GLOBAL float* v = (OPT_GLOBAL float*)exp_avg_sq[t];
  const OPT_GLOBAL G* g = (const OPT_GLOBAL G*)reinterpret_cast<const G*>(grads[t]);
  const bool separate = (const OPT_GLOBAL void*)w != (const OPT_GLOBAL void*)p;
  auto update = [&](float gi, float& wi, float& mi, float& vi) {
    gi *= clip;
    wi *= decay;
    mi = mi + (1.0f - beta1) * (gi - mi);
    vi = vi * beta2 + (1.0f - beta2) * gi * gi;
    const float denom = sqrtf(vi) / bc2_sqrt + eps;
    wi = wi - step_size * (mi / denom);
  };
  int64_t i = beg;
  // float32 state 16-byte aligned; 4 gradient / parameter elements are 16
  // bytes (float) or 8 bytes (bf16)
  constexpr uintptr_t half = sizeof(T) == 2 ? 2 : 1;
  constexpr uintptr_t ghalf = sizeof(G) == 2 ? 2 : 1;
  const uintptr_t align = (uintptr_t)(w + beg) | (uintptr_t)(m + beg) | (uintptr_t)(v + beg) |
                          (uintptr_t)(g + beg) * ghalf | (separate ? (uintptr_t)(p + beg) * half : 0);
  if ((align & 15) == 0) {
    // 4 elements per thread and group: 16-byte float32 state, 4 * sizeof(T)
    // bytes of gradient and parameter (the same arithmetic per element).  Two
    // groups per step, all their loads issued before either is updated (the
    // stores would otherwise order every load after the previous group's
    // stores), and every stream non-temporal: each byte is read and written
    // once.
    const int64_t vec_end = beg + (end - beg) / 4 * 4;
    constexpr int64_t STRIDE = OPT_THREADS * 4;
    typedef float nt_f4 __attribute__((ext_vector_type(4)));
    typedef unsigned nt_u2 __attribute__((ext_vector_type(2)));
    auto load4f = [](const OPT_GLOBAL float* a) {
      const nt_f4 q = __builtin_nontemporal_load((const OPT_GLOBAL nt_f4*)a);
      return make_float4(q.x, q.y, q.z, q.w);
    };
    auto store4f = [](OPT_GLOBAL float* a, float x, float y, float z, float wv) {
      __builtin_nontemporal_store(nt_f4{x, y, z, wv}, (OPT_GLOBAL nt_f4*)a);
    };
    auto load_g = [&](int64_t j, float* gv) {
      if constexpr (sizeof(G) == 2) {
        const nt_u2 gr = __builtin_nontemporal_load((const OPT_GLOBAL nt_u2*)(g + j));
        gv[0] = bf16_to_float((bf16_t)(gr.x & 0xffff)); gv[1] = bf16_to_float((bf16_t)(gr.x >> 16));
        gv[2] = bf16_to_float((bf16_t)(gr.y & 0xffff)); gv[3] = bf16_to_float((bf16_t)(gr.y >> 16));
      } else {
        const float4 g4 = load4f((const OPT_GLOBAL float*)g + j);
        gv[0] = g4.x; gv[1] = g4.y; gv[2] = g4.z; gv[3] = g4.w;
      }
    };
    auto finish = [&](int64_t j, float* gv, float4 w4, float4 m4, float4 v4) {
      float wv[4] = {w4.x, w4.y, w4.z, w4.w}, mv[4] = {m4.x, m4.y, m4.z, m4.w},
            vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) update(gv[e], wv[e], mv[e], vv[e]);
      store4f(m + j, mv[0], mv[1], mv[2], mv[3]);
      store4f(v + j, vv[0], vv[1], vv[2], vv[3]);
      store4f(w + j, wv[0], wv[1], wv[2], wv[3]);
      if (separate) {
        if constexpr (sizeof(T) == 2) {
          __builtin_nontemporal_store(nt_u2{pack_bf16x2(wv[0], wv[1]), pack_bf16x2(wv[2], wv[3])},
                                      (OPT_GLOBAL nt_u2*)(p + j));
        } else {
          store4f((OPT_GLOBAL float*)p + j, wv[0], wv[1], wv[2], wv[3]);
        }
      }
    };
    int64_t j = beg + threadIdx.x * 4;
    for (; j + STRIDE < vec_end; j += 2 * STRIDE) {
      const int64_t j2 = j + STRIDE;
      float ga[4], gb[4];
      const float4 wa = load4f(w + j), ma = load4f(m + j), va = load4f(v + j);
      const float4 wb = load4f(w + j2), mb = load4f(m + j2), vb = load4f(v + j2);
      load_g(j, ga);
      load_g(j2, gb);
      finish(j, ga, wa, ma, va);
      finish(j2, gb, wb, mb, vb);
    }
    if (j < vec_end) {
      float ga[4];
      const float4 wa = load4f(w + j), ma = load4f(m + j), va = load4f(v + j);
      load_g(j, ga);
      finish(j, ga, wa, ma, va);
    }
    i = vec_end;
  }
  for (i += threadIdx.x; i < end; i += OPT_THREADS) {
    float wi = w[i], mi = m[i], vi = v[i];
    update(Elem<G>::load((const G*)g, i), wi, mi, vi);
    m[i] = mi;
    v[i] = vi;
    w[i] = wi;
    if (separate) Elem<T>::store((T*)p, i, wi);
  }
}

extern "C" int alodlm_grad_norm(const void* const* grads, const int32_t* chunk_tensor,
                                const int64_t* chunk_start, const int64_t* numels,
                                int64_t n_chunks, int64_t chunk_size, int dtype, float* partial,
                                float* total_norm, void* stream) {
  ALODLM_CHECK_ARG(n_chunks > 0 && chunk_size > 0, "grad_norm: empty tensor list");
  hipStream_t st = as_stream(stream);
  ALODLM_DISPATCH(dtype, T, {
    grad_sumsq_kernel<T><<<(unsigned)n_chunks, OPT_THREADS, 0, st>>>(
        grads, chunk_tensor, chunk_start, numels, chunk_size, partial);
  });
  ALODLM_CHECK_LAUNCH("grad_sumsq");
  final_norm_kernel<<<1, 1024, 0, st>>>(partial, n_chunks, total_norm);
  ALODLM_CHECK_LAUNCH("grad_norm_final");
  return ALODLM_OK;
}

extern "C" int alodlm_adamw(void* const* params, float* const* master, float* const* exp_avg,
                            float* const* exp_avg_sq, const void* const* grads,
                            const int32_t* chunk_tensor, const int64_t* chunk_start,
                            const int64_t* numels, const float* weight_decay, int64_t n_chunks,
                            int64_t chunk_size, const float* total_norm, float max_norm, float lr,
                            float beta1, float beta2, float eps, int64_t step, int dtype,
                            int grad_dtype, void* stream) {
  ALODLM_CHECK_ARG(n_chunks > 0 && chunk_size > 0, "adamw: empty tensor list");
  ALODLM_CHECK_ARG(step >= 1, "adamw: step must be >= 1");
  const double bc1 = 1.0 - pow((double)beta1, (double)step);
  const double bc2 = 1.0 - pow((double)beta2, (double)step);
  const float step_size = (float)((double)lr / bc1);
  const float bc2_sqrt = (float)sqrt(bc2);
  ALODLM_CHECK_ARG(grad_dtype == dtype || grad_dtype == ALODLM_F32,
                   "adamw: gradients are float32 or of the parameter dtype");
  ALODLM_DISPATCH(dtype, T, {
    if (grad_dtype == ALODLM_F32)
      adamw_kernel<T, float><<<(unsigned)n_chunks, OPT_THREADS, 0, as_stream(stream)>>>(
          params, master, exp_avg, exp_avg_sq, grads, chunk_tensor, chunk_start, numels,
          weight_decay, chunk_size, total_norm, max_norm, lr, beta1, beta2, eps, step_size,
          bc2_sqrt);
    else
      adamw_kernel<T, T><<<(unsigned)n_chunks, OPT_THREADS, 0, as_stream(stream)>>>(
          params, master, exp_avg, exp_avg_sq, grads, chunk_tensor, chunk_start, numels,
          weight_decay, chunk_size, total_norm, max_norm, lr, beta1, beta2, eps, step_size,
          bc2_sqrt);
  });
  ALODLM_CHECK_LAUNCH("adamw");
  return ALODLM_OK;
}
