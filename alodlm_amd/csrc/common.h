// Shared device helpers for the ALoDLM gfx950 kernels.
//
// Storage types: float (dtype code 0) and bfloat16 held as uint16_t (dtype
// code 1).  All arithmetic is float32; bf16 results are rounded to nearest
// even exactly once per reference rounding point, so that bf16 runs follow
// the reference's bf16 eager rounding sequence.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/alodlm_hip.h"

typedef uint16_t bf16_t;

#define ALODLM_WAVE 64

// ----------------------------------------------------------------------------
// bf16 <-> float
// ----------------------------------------------------------------------------
__host__ __device__ __forceinline__ float bf16_to_float(bf16_t h) {
  union { uint32_t u; float f; } v;
  v.u = (uint32_t)h << 16;
  return v.f;
}

// Round to nearest even (gfx950: one v_cvt_pk_bf16_f32 per pair of values).
__device__ __forceinline__ bf16_t float_to_bf16(float f) {
  return __builtin_bit_cast(bf16_t, (__bf16)f);
}

// Two floats rounded to nearest-even bf16, `lo` in the low half: one
// v_cvt_pk_bf16_f32 with both sources (two scalar conversions OR-ed together
// compile to two conversions plus the shift and the OR).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_v __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  const f32x2_v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_v));
}

// Round a float to the nearest bf16 value and return it as float.
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_float(float_to_bf16(f)); }

template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
  // Rounding to the storage precision (identity for float).
  static __device__ __forceinline__ float round(float v) { return v; }
};
template <> struct Elem<bf16_t> {
  static __device__ __forceinline__ float load(const bf16_t* p, int64_t i) { return bf16_to_float(p[i]); }
  static __device__ __forceinline__ void store(bf16_t* p, int64_t i, float v) { p[i] = float_to_bf16(v); }
  static __device__ __forceinline__ float round(float v) { return round_bf16(v); }
};

// ----------------------------------------------------------------------------
// Wavefront / block reductions (64-wide wavefronts)
// ----------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum over the whole block; every thread gets the result.  `scratch` must
// hold blockDim.x/64 floats.  Deterministic (fixed tree order).
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.f;
  for (int w = 0; w < nwaves; ++w) total += scratch[w];
  return total;
}

__device__ __forceinline__ float block_max(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = -INFINITY;
  for (int w = 0; w < nwaves; ++w) total = fmaxf(total, scratch[w]);
  return total;
}

__device__ __forceinline__ float sigmoidf_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// softplus(x) = log(1 + exp(x)) with torch's threshold of 20.
__device__ __forceinline__ float softplusf(float x) { return x > 20.f ? x : log1pf(expf(x)); }

// ----------------------------------------------------------------------------
// Host-side error plumbing (defined in abi.hip)
// ----------------------------------------------------------------------------
int alodlm_set_error(int code, const char* fmt, ...);

#define ALODLM_CHECK_ARG(cond, ...)                                  \
  do {                                                               \
    if (!(cond)) return alodlm_set_error(ALODLM_EINVAL, __VA_ARGS__); \
  } while (0)

#define ALODLM_CHECK_LAUNCH(name)                                                   \
  do {                                                                              \
    hipError_t _e = hipGetLastError();                                              \
    if (_e != hipSuccess)                                                           \
      return alodlm_set_error(ALODLM_EHIP, "%s: %s", name, hipGetErrorString(_e));  \
  } while (0)

static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Number of blocks of b threads covering a items.  A dispatch holds fewer
// than 2^32 work-items in each dimension, so every caller's a is bounded by
// the activation shapes (or the kernel is a grid-stride sweep).
static inline unsigned ceil_div_u(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// Compute units of the current device, cached per device (grids of one
// workgroup per CU).
static inline int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev]) return cached[dev];
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  if (dev < 64) cached[dev] = cus;
  return cus;
}

// ----------------------------------------------------------------------------
// 8-element vector access (16 bytes of bf16 or 32 bytes of float).  The
// pointer must be aligned to 8 elements.
// ----------------------------------------------------------------------------
// 8 consecutive elements as floats.  load_nt / store_nt are the same accesses
// marked non-temporal, for streams read or written once that are much larger
// than the caches.
typedef unsigned nt_u32x4_t __attribute__((ext_vector_type(4)));
typedef float nt_f32x4_t __attribute__((ext_vector_type(4)));
template <typename T> struct Vec8;
template <> struct Vec8<bf16_t> {
  static __device__ __forceinline__ void unpack(const uint32_t* w, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_to_float((bf16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = bf16_to_float((bf16_t)(w[i] >> 16));
    }
  }
  static __device__ __forceinline__ void load(const bf16_t* p, float* v) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
    unpack(w, v);
  }
  static __device__ __forceinline__ void load_nt(const bf16_t* p, float* v) {
    const nt_u32x4_t u = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4_t*>(p));
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
    unpack(w, v);
  }
  static __device__ __forceinline__ void store(bf16_t* p, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  static __device__ __forceinline__ void store_nt(bf16_t* p, const float* v) {
    nt_u32x4_t w;
    w.x = pack_bf16x2(v[0], v[1]);
    w.y = pack_bf16x2(v[2], v[3]);
    w.z = pack_bf16x2(v[4], v[5]);
    w.w = pack_bf16x2(v[6], v[7]);
    __builtin_nontemporal_store(w, reinterpret_cast<nt_u32x4_t*>(p));
  }
};
template <> struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    float4 a = reinterpret_cast<const float4*>(p)[0];
    float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void load_nt(const float* p, float* v) {
    const nt_f32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4_t*>(p));
    const nt_f32x4_t b = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4_t*>(p) + 1);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
  static __device__ __forceinline__ void store_nt(float* p, const float* v) {
    __builtin_nontemporal_store(nt_f32x4_t{v[0], v[1], v[2], v[3]},
                                reinterpret_cast<nt_f32x4_t*>(p));
    __builtin_nontemporal_store(nt_f32x4_t{v[4], v[5], v[6], v[7]},
                                reinterpret_cast<nt_f32x4_t*>(p) + 1);
  }
};

static inline bool aligned8(const void* p, int dtype) {
  return (reinterpret_cast<uintptr_t>(p) % (dtype == ALODLM_BF16 ? 16 : 32)) == 0;
}

// Dispatch a templated launcher over the storage type.
#define ALODLM_DISPATCH(dtype, T, ...)                                        \
  do {                                                                        \
    if ((dtype) == ALODLM_F32) { typedef float T; __VA_ARGS__; }              \
    else if ((dtype) == ALODLM_BF16) { typedef bf16_t T; __VA_ARGS__; }       \
    else return alodlm_set_error(ALODLM_EINVAL, "unknown dtype %d", (int)(dtype)); \
  } while (0)
