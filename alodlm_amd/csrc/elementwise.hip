// Embedding gather, SwiGLU, and small elementwise helpers.
#include "common.h"

// out[r] = table[ids[r]]   ([tf] modeling_qwen3.py:352; alodlm/model.py:133,149)
// An id outside [0, vocab) yields a NaN row instead of an out-of-bounds read.
template <typename T>
__global__ void embed_gather_kernel(const T* __restrict__ table, const int64_t* __restrict__ ids,
                                    T* __restrict__ out, int64_t rows, int64_t H, int64_t vocab) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * H) return;
  const int64_t r = i / H, c = i % H;
  const int64_t id = ids[r];
  if (id < 0 || id >= vocab) Elem<T>::store(out, i, NAN);
  else out[i] = table[id * H + c];
}

// act = cast(cast(silu(gate)) * up)   ([tf] modeling_qwen3.py:81-83).
// gu rows are [gate | up] of width 2I; W elements per thread (8 with 16-byte
// vector access when I % 8 == 0, else 1).
template <typename T, int W>
__global__ void swiglu_fwd_kernel(const T* __restrict__ gu, T* __restrict__ act, int64_t rows,
                                  int64_t I) {
  // W == 8: 8-column groups along grid x, one row per grid y (blocks are
  // dispatched x first, so the streams stay sequential; the flat grid's
  // 64-bit division for the row and column was 170 of 466 instructions:
  // 206.7 -> 187.8 us per 1.7B call); W == 1: a flat grid
  int64_t r, c;
  if (W == 8) {
    r = blockIdx.y;
    c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (c >= I) return;
  } else {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * I) return;
    r = i / I;
    c = i % I;
  }
  const int64_t i = r * I + c;
  float g[8], u[8], a[8];
  // the streams are far larger than the caches and used once here: non-temporal
  if (W == 8) {
    Vec8<T>::load_nt(gu + r * 2 * I + c, g);
    Vec8<T>::load_nt(gu + r * 2 * I + I + c, u);
  } else {
    g[0] = Elem<T>::load(gu, r * 2 * I + c);
    u[0] = Elem<T>::load(gu, r * 2 * I + I + c);
  }
#pragma unroll
  for (int e = 0; e < W; ++e) a[e] = Elem<T>::round(g[e] / (1.0f + expf(-g[e]))) * u[e];
  if (W == 8) Vec8<T>::store_nt(act + i, a);
  else Elem<T>::store(act, i, a[0]);
}

// dgate = dact * up * silu'(gate), dup = dact * silu(gate); where act is not
// null the forward product act = cast(cast(silu(gate)) * up) is written too
// (the same expression as swiglu_fwd_kernel, so the value is bit-identical),
// which saves the backward a separate recompute pass over gu.
template <typename T, int W>
__global__ void swiglu_bwd_kernel(const T* __restrict__ dact, const T* __restrict__ gu,
                                  T* __restrict__ dgu, T* __restrict__ act, int64_t rows,
                                  int64_t I) {
  int64_t r, c;  // the grid of swiglu_fwd_kernel
  if (W == 8) {
    r = blockIdx.y;
    c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (c >= I) return;
  } else {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * I) return;
    r = i / I;
    c = i % I;
  }
  const int64_t i = r * I + c;
  float g[8], u[8], da[8], dg[8], du[8], a[8];
  if (W == 8) {
    Vec8<T>::load_nt(gu + r * 2 * I + c, g);
    Vec8<T>::load_nt(gu + r * 2 * I + I + c, u);
    Vec8<T>::load_nt(dact + i, da);
  } else {
    g[0] = Elem<T>::load(gu, r * 2 * I + c);
    u[0] = Elem<T>::load(gu, r * 2 * I + I + c);
    da[0] = Elem<T>::load(dact, i);
  }
#pragma unroll
  for (int e = 0; e < W; ++e) {
    const float sg = 1.0f / (1.0f + expf(-g[e]));
    dg[e] = da[e] * u[e] * (sg * (1.0f + g[e] * (1.0f - sg)));
    du[e] = da[e] * Elem<T>::round(g[e] * sg);
    a[e] = Elem<T>::round(g[e] / (1.0f + expf(-g[e]))) * u[e];
  }
  if (W == 8) {
    Vec8<T>::store_nt(dgu + r * 2 * I + c, dg);
    Vec8<T>::store_nt(dgu + r * 2 * I + I + c, du);
    if (act) Vec8<T>::store_nt(act + i, a);
  } else {
    Elem<T>::store(dgu, r * 2 * I + c, dg[0]);
    Elem<T>::store(dgu, r * 2 * I + I + c, du[0]);
    if (act) Elem<T>::store(act, i, a[0]);
  }
}

// dst[c][r] = src[r][c] for a rows x cols matrix, through a 64 x 64 LDS tile
// (row pitch 65 elements, so the column reads of the transposed pass fall in
// distinct banks).  One workgroup of 256 threads per tile.
template <typename T>
__global__ void __launch_bounds__(256)
transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t rows, int64_t cols) {
  __shared__ T tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rr = ty + 4 * i;
    const int64_t r = r0 + rr, c = c0 + tx;
    if (r < rows && c < cols) tile[rr][tx] = src[r * cols + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int cc = ty + 4 * i;
    const int64_t c = c0 + cc, r = r0 + tx;
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][cc];
  }
}

// The same transpose for 2-byte elements with rows and cols multiples of 8
// and 16-byte aligned rows: 64x64 tiles moved in 16-byte pieces.  On the
// way in, 8 threads per tile row; on the way out each thread reads 8 tile
// rows x 2 columns as 32-bit words and writes two transposed 16-byte pieces
// (half the LDS reads of one column per thread).  Word w of tile row r sits
// at w ^ 8 * ((r / 16) % 4): the 64 lanes of a read (8 row groups x 8 word
// columns) then fall in 64 distinct banks, and the 16-byte pieces written on
// the way in stay contiguous.
__global__ void __launch_bounds__(256)
transpose16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst, int64_t rows,
                   int64_t cols) {
  __shared__ uint32_t tile[64][32];  // [row][word] (2 elements per word)
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
  auto sw = [](int r) { return 8 * ((r >> 4) & 3); };
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int rr = (t >> 3) + 32 * pass, part = (t & 7) * 8;
    const int64_t r = r0 + rr, c = c0 + part;
    if (r < rows && c < cols)
      *reinterpret_cast<uint4*>(&tile[rr][(part / 2) ^ sw(rr)]) =
          *reinterpret_cast<const uint4*>(src + r * cols + c);
  }
  __syncthreads();
  const int part = (t & 7) * 8;  // 8 tile rows part .. part + 7
  const int cc = (t >> 3) * 2;   // tile columns cc, cc + 1
  const int64_t r = r0 + part, c = c0 + cc;
  if (r < rows && c < cols) {
    uint32_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = tile[part + k][(cc / 2) ^ sw(part + k)];
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[e] = (v[2 * e] & 0xffffu) | (v[2 * e + 1] << 16);          // column cc
      hi[e] = (v[2 * e] >> 16) | (v[2 * e + 1] & 0xffff0000u);      // column cc + 1
    }
    *reinterpret_cast<uint4*>(dst + c * rows + r) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    if (c + 1 < cols)
      *reinterpret_cast<uint4*>(dst + (c + 1) * rows + r) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  }
}

// dst = cast(src * scale[0]) (scale may be null: no scaling).  Grid-stride:
// these two kernels sweep the whole gradient arena (8.2 G elements at 8B), and
// one dispatch covers fewer than 2^32 work-items.
template <typename T>
__global__ void cast_kernel(const float* __restrict__ src, const float* __restrict__ scale,
                            T* __restrict__ dst, int64_t n) {
  const float k = scale ? scale[0] : 1.0f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t head = 0;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 31) == 0) {
    // 8 elements per thread and step: two 16-byte float loads, one store of
    // 8 * sizeof(T) bytes; the tail below takes the rest
    head = n / 8 * 8;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < head; i += stride * 8) {
      float v[8];
      Vec8<float>::load(src + i, v);
      if (scale) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] *= k;
      }
      Vec8<T>::store(dst + i, v);
    }
  }
  for (int64_t i = head + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    Elem<T>::store(dst, i, scale ? src[i] * k : src[i]);
}

__global__ void scale_kernel(float* __restrict__ x, const float* __restrict__ s, int64_t n) {
  const float k = s[0];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) x[i] *= k;
}

// x *= s[0] in the storage dtype (rounded once per element).
template <typename T>
__global__ void scale_any_kernel(T* __restrict__ x, const float* __restrict__ s, int64_t n) {
  const float k = s[0];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t head = 0;
  if (reinterpret_cast<uintptr_t>(x) % 16 == 0 && 16 % sizeof(T) == 0) {
    // 16 bytes per thread and step (8 or 4 elements); the tail below
    constexpr int PER = 16 / sizeof(T);
    head = n / PER * PER;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * PER; i < head;
         i += stride * PER) {
      T e[PER];
      *reinterpret_cast<uint4*>(e) = *reinterpret_cast<const uint4*>(x + i);
#pragma unroll
      for (int q = 0; q < PER; ++q) Elem<T>::store(e, q, Elem<T>::load(e, q) * k);
      *reinterpret_cast<uint4*>(x + i) = *reinterpret_cast<const uint4*>(e);
    }
  }
  for (int64_t i = head + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    Elem<T>::store(x, i, Elem<T>::load(x, i) * k);
}

// y = s[0] * x + (accumulate ? y : 0) in float32, four elements per thread
// and step where both are 16-byte aligned (the tail takes the rest).
__global__ void scale_add_kernel(const float* __restrict__ x, float* __restrict__ y,
                                 const float* __restrict__ s, int64_t n, int accumulate) {
  const float k = s ? s[0] : 1.0f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t head = 0;
  if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0) {
    head = n / 4 * 4;
    for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < head;
         i += stride * 4) {
      const float4 a = *reinterpret_cast<const float4*>(x + i);
      float4 b = accumulate ? *reinterpret_cast<const float4*>(y + i) : make_float4(0, 0, 0, 0);
      b.x += k * a.x;
      b.y += k * a.y;
      b.z += k * a.z;
      b.w += k * a.w;
      *reinterpret_cast<float4*>(y + i) = b;
    }
  }
  for (int64_t i = head + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (accumulate ? y[i] : 0.0f) + k * x[i];
}

// Blocks of 256 for a grid-stride sweep over n elements (at most 8 per CU slot
// of a 256-CU part, so the grid stays far below the 2^32 work-item limit).
static unsigned sweep_blocks(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return (unsigned)(b < 16384 ? b : 16384);
}

extern "C" int alodlm_embed_gather(const void* table, const int64_t* ids, void* out, int64_t rows,
                                   int64_t hidden, int64_t vocab, int dtype, void* stream) {
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    embed_gather_kernel<T><<<ceil_div_u(rows * hidden, 256), 256, 0, as_stream(stream)>>>(
        (const T*)table, ids, (T*)out, rows, hidden, vocab);
  });
  ALODLM_CHECK_LAUNCH("embed_gather");
  return ALODLM_OK;
}

extern "C" int alodlm_swiglu_fwd(const void* gu, void* act, int64_t rows, int64_t inter, int dtype,
                                 void* stream) {
  if (rows == 0) return ALODLM_OK;
  const bool v8 = inter % 8 == 0 && aligned8(gu, dtype) && aligned8(act, dtype);
  ALODLM_DISPATCH(dtype, T, {
    if (v8)
      // one row per grid y: launches of at most 65535 rows
      for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        const int64_t n = rows - r0 < 65535 ? rows - r0 : 65535;
        swiglu_fwd_kernel<T, 8><<<dim3(ceil_div_u(inter / 8, 256), (unsigned)n), 256, 0,
                                  as_stream(stream)>>>((const T*)gu + r0 * 2 * inter,
                                                       (T*)act + r0 * inter, n, inter);
      }
    else
      swiglu_fwd_kernel<T, 1><<<ceil_div_u(rows * inter, 256), 256, 0, as_stream(stream)>>>(
          (const T*)gu, (T*)act, rows, inter);
  });
  ALODLM_CHECK_LAUNCH("swiglu_fwd");
  return ALODLM_OK;
}

extern "C" int alodlm_swiglu_bwd(const void* dact, const void* gu, void* dgu, void* act,
                                 int64_t rows, int64_t inter, int dtype, void* stream) {
  if (rows == 0) return ALODLM_OK;
  const bool v8 = inter % 8 == 0 && aligned8(gu, dtype) && aligned8(dact, dtype) &&
                  aligned8(dgu, dtype) && (act == nullptr || aligned8(act, dtype));
  ALODLM_DISPATCH(dtype, T, {
    if (v8)
      for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
        const int64_t n = rows - r0 < 65535 ? rows - r0 : 65535;
        swiglu_bwd_kernel<T, 8><<<dim3(ceil_div_u(inter / 8, 256), (unsigned)n), 256, 0,
                                  as_stream(stream)>>>(
            (const T*)dact + r0 * inter, (const T*)gu + r0 * 2 * inter,
            (T*)dgu + r0 * 2 * inter, act ? (T*)act + r0 * inter : nullptr, n, inter);
      }
    else
      swiglu_bwd_kernel<T, 1><<<ceil_div_u(rows * inter, 256), 256, 0, as_stream(stream)>>>(
          (const T*)dact, (const T*)gu, (T*)dgu, (T*)act, rows, inter);
  });
  ALODLM_CHECK_LAUNCH("swiglu_bwd");
  return ALODLM_OK;
}

extern "C" int alodlm_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int dtype,
                                void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && cols >= 0, "transpose: negative shape");
  ALODLM_CHECK_ARG(rows <= 64 * 65535LL, "transpose: too many rows");
  if (rows == 0 || cols == 0) return ALODLM_OK;
  ALODLM_CHECK_ARG(src != dst, "transpose: in-place transpose is not supported");
  dim3 grid(ceil_div_u(cols, 64), ceil_div_u(rows, 64));
  if (dtype == ALODLM_BF16 && rows % 8 == 0 && cols % 8 == 0 &&
      ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
    transpose16_kernel<<<grid, 256, 0, as_stream(stream)>>>((const uint16_t*)src, (uint16_t*)dst,
                                                            rows, cols);
    ALODLM_CHECK_LAUNCH("transpose");
    return ALODLM_OK;
  }
  ALODLM_DISPATCH(dtype, T, {
    transpose_kernel<T><<<grid, 256, 0, as_stream(stream)>>>((const T*)src, (T*)dst, rows, cols);
  });
  ALODLM_CHECK_LAUNCH("transpose");
  return ALODLM_OK;
}

// *flag = 1 when any of the n elements is inf or NaN (read once, 16 bytes per
// thread and step of a grid-stride sweep; the flag is only ever set, by a
// vector store of the same value).
template <typename T>
__global__ void __launch_bounds__(256)
check_finite_kernel(const T* __restrict__ x, int64_t n, int32_t* __restrict__ flag) {
  constexpr int PER = 16 / sizeof(T);
  const int64_t stride = (int64_t)gridDim.x * 256 * PER;
  bool bad = false;
  int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * PER;
  if (reinterpret_cast<uintptr_t>(x) % 16 == 0) {
    for (; i + PER <= n; i += stride) {
      const nt_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4_t*>(x + i));
      T e[PER];
      __builtin_memcpy(e, &v, 16);
#pragma unroll
      for (int k = 0; k < PER; ++k) bad |= !isfinite(Elem<T>::load(e, k));
    }
  }
  for (; i < n; i += stride)  // the tail (or an unaligned array) element by element
    for (int k = 0; k < PER && i + k < n; ++k) bad |= !isfinite(Elem<T>::load(x, i + k));
  if (bad) *flag = 1;
}

extern "C" int alodlm_check_finite(const void* x, int64_t n, int dtype, int32_t* flag,
                                   void* stream) {
  ALODLM_CHECK_ARG(n >= 0, "check_finite: negative size");
  ALODLM_CHECK_ARG(flag != nullptr, "check_finite: no flag");
  if (n == 0) return ALODLM_OK;
  const unsigned blocks = (unsigned)std::min<int64_t>(4 * (int64_t)device_cus(), ceil_div_u(n, 256 * 8));
  ALODLM_DISPATCH(dtype, T, {
    check_finite_kernel<T><<<blocks, 256, 0, as_stream(stream)>>>((const T*)x, n, flag);
  });
  ALODLM_CHECK_LAUNCH("check_finite");
  return ALODLM_OK;
}

extern "C" int alodlm_cast_f32(const float* src, const float* scale, void* dst, int64_t n,
                               int dtype, void* stream) {
  if (n == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    cast_kernel<T><<<sweep_blocks(n), 256, 0, as_stream(stream)>>>(src, scale, (T*)dst, n);
  });
  ALODLM_CHECK_LAUNCH("cast_f32");
  return ALODLM_OK;
}

extern "C" int alodlm_scale_f32(float* x, const float* scale, int64_t n, void* stream) {
  if (n == 0) return ALODLM_OK;
  scale_kernel<<<sweep_blocks(n), 256, 0, as_stream(stream)>>>(x, scale, n);
  ALODLM_CHECK_LAUNCH("scale_f32");
  return ALODLM_OK;
}

extern "C" int alodlm_scale(void* x, const float* scale, int64_t n, int dtype, void* stream) {
  ALODLM_CHECK_ARG(n >= 0 && scale != nullptr, "scale: bad arguments");
  if (n == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    scale_any_kernel<T><<<sweep_blocks(n), 256, 0, as_stream(stream)>>>((T*)x, scale, n);
  });
  ALODLM_CHECK_LAUNCH("scale");
  return ALODLM_OK;
}

extern "C" int alodlm_scale_add_f32(const float* x, float* y, int64_t n, const float* scale,
                                    int accumulate, void* stream) {
  ALODLM_CHECK_ARG(n >= 0, "scale_add_f32: negative size");
  if (n == 0) return ALODLM_OK;
  scale_add_kernel<<<sweep_blocks((n + 3) / 4), 256, 0, as_stream(stream)>>>(x, y, scale, n,
                                                                              accumulate);
  ALODLM_CHECK_LAUNCH("scale_add_f32");
  return ALODLM_OK;
}
