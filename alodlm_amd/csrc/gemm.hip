// GEMM for every linear layer of the step.
//
//   C[m, n] = alpha * sum_k A(m, k) * B(n, k)
//
// bf16 path: 128x128x64 tiles, 4 wavefronts in a 2x2 grid, each computing a
// 64x64 block with v_mfma_f32_32x32x16_bf16.  Operands are staged through LDS
// in k-contiguous rows (padded by 8 elements); an operand stored m/n-contiguous
// ([K, M] in memory, as in the backward's dW and dX products) is transposed
// while it is staged: each thread loads an 8(k) x 4(m) block with 8-byte
// loads and writes four 16-byte k-rows.  Global loads for tile k+1 are issued
// before the MFMAs of tile k (register prefetch, double-buffered LDS).
//
// float path and unaligned shapes: a plain LDS-tiled FMA kernel.
#include "common.h"
#include "gemm_dl.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

#define GM_BM 128
#define GM_BN 128
#define GM_BK 64
#define GM_LDK (GM_BK + 8)  // padded LDS row (elements)
#define GM_THREADS 256

// ---------------------------------------------------------------------------
// Global -> register staging of one operand tile (rows x 64 k)
// ---------------------------------------------------------------------------
struct StageK {  // k-contiguous operand: 4 chunks of 8 elements per thread
  uint4 v[4];
};
struct StageMN {  // m/n-contiguous operand: 8 k-rows x 4 elements per thread
  uint2 v[8];
};

__device__ __forceinline__ void load_kmajor(const bf16_t* __restrict__ P, int64_t ld, int64_t r0,
                                            int64_t rows, int64_t k0, int64_t K, StageK& s) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + GM_THREADS * i;
    const int row = c >> 3, kc = (c & 7) * 8;
    const int64_t gr = r0 + row, gk = k0 + kc;
    if (gr < rows && gk + 8 <= K)
      s.v[i] = *reinterpret_cast<const uint4*>(P + gr * ld + gk);
    else
      s.v[i] = make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void store_kmajor(bf16_t* lds, const StageK& s) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = threadIdx.x + GM_THREADS * i;
    const int row = c >> 3, kc = (c & 7) * 8;
    *reinterpret_cast<uint4*>(lds + row * GM_LDK + kc) = s.v[i];
  }
}

__device__ __forceinline__ void load_mnmajor(const bf16_t* __restrict__ P, int64_t ld, int64_t r0,
                                             int64_t rows, int64_t k0, int64_t K, StageMN& s) {
  const int rq = threadIdx.x & 31, kq = threadIdx.x >> 5;
  const int64_t gr = r0 + rq * 4;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t gk = k0 + kq * 8 + j;
    if (gk < K && gr + 4 <= rows)
      s.v[j] = *reinterpret_cast<const uint2*>(P + gk * ld + gr);
    else
      s.v[j] = make_uint2(0, 0);
  }
}

__device__ __forceinline__ void store_mnmajor(bf16_t* lds, const StageMN& s) {
  const int rq = threadIdx.x & 31, kq = threadIdx.x >> 5;
  // element (k=j, r) sits in s.v[j].{x: r0|r1<<16, y: r2|r3<<16}
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t a = (r < 2) ? s.v[2 * p].x : s.v[2 * p].y;
      const uint32_t b = (r < 2) ? s.v[2 * p + 1].x : s.v[2 * p + 1].y;
      w[p] = (r & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    *reinterpret_cast<uint4*>(lds + (rq * 4 + r) * GM_LDK + kq * 8) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <bool AK> struct StageOf { typedef StageK type; };
template <> struct StageOf<false> { typedef StageMN type; };

template <bool KMAJOR>
__device__ __forceinline__ void load_tile(const bf16_t* P, int64_t ld, int64_t r0, int64_t rows,
                                          int64_t k0, int64_t K, typename StageOf<KMAJOR>::type& s);
template <>
__device__ __forceinline__ void load_tile<true>(const bf16_t* P, int64_t ld, int64_t r0, int64_t rows,
                                                int64_t k0, int64_t K, StageK& s) {
  load_kmajor(P, ld, r0, rows, k0, K, s);
}
template <>
__device__ __forceinline__ void load_tile<false>(const bf16_t* P, int64_t ld, int64_t r0,
                                                 int64_t rows, int64_t k0, int64_t K, StageMN& s) {
  load_mnmajor(P, ld, r0, rows, k0, K, s);
}
__device__ __forceinline__ void store_tile(bf16_t* lds, const StageK& s) { store_kmajor(lds, s); }
__device__ __forceinline__ void store_tile(bf16_t* lds, const StageMN& s) { store_mnmajor(lds, s); }

// ---------------------------------------------------------------------------
// bf16 MFMA kernel
// ---------------------------------------------------------------------------
template <bool AK, bool BK, int EPI>
__global__ void __launch_bounds__(GM_THREADS, 2)
gemm_bf16_kernel(const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ B,
                 int64_t ldb, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                 int64_t N, int64_t K, float alpha, int64_t k_per_split, float* __restrict__ partial) {
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][GM_BM * GM_LDK];  // [buf][A/B]

  // tile order: groups of 8 tile-rows sweep the tile-columns (L2 reuse of B)
  const int64_t tiles_m = (M + GM_BM - 1) / GM_BM, tiles_n = (N + GM_BN - 1) / GM_BN;
  const int64_t tid = blockIdx.x;
  const int64_t group = 8;
  const int64_t per_group = group * tiles_n;
  const int64_t g = tid / per_group;
  const int64_t first_m = g * group;
  const int64_t gsize = (tiles_m - first_m) < group ? (tiles_m - first_m) : group;
  const int64_t tm = first_m + (tid % per_group) % gsize;
  const int64_t tn = (tid % per_group) / gsize;
  const int64_t m0 = tm * GM_BM, n0 = tn * GM_BN;
  const int64_t kbeg = (int64_t)blockIdx.y * k_per_split;
  const int64_t kend = (kbeg + k_per_split) < K ? (kbeg + k_per_split) : K;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  typename StageOf<AK>::type sa;
  typename StageOf<BK>::type sb;
  int buf = 0;
  if (kbeg < kend) {
    load_tile<AK>(A, lda, m0, M, kbeg, kend, sa);
    load_tile<BK>(B, ldb, n0, N, kbeg, kend, sb);
    store_tile(lds[0][0], sa);
    store_tile(lds[0][1], sb);
  }
  __syncthreads();
  for (int64_t k0 = kbeg; k0 < kend; k0 += GM_BK) {
    const bool more = k0 + GM_BK < kend;
    if (more) {
      load_tile<AK>(A, lda, m0, M, k0 + GM_BK, kend, sa);
      load_tile<BK>(B, ldb, n0, N, k0 + GM_BK, kend, sb);
    }
    const bf16_t* la = lds[buf][0];
    const bf16_t* lb = lds[buf][1];
#pragma unroll
    for (int ks = 0; ks < GM_BK; ks += 16) {
      bf16x8_t fa[2], fb[2];
      const int kk = ks + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        fa[i] = *reinterpret_cast<const bf16x8_t*>(la + (wm * 64 + i * 32 + (lane & 31)) * GM_LDK + kk);
        fb[i] = *reinterpret_cast<const bf16x8_t*>(lb + (wn * 64 + i * 32 + (lane & 31)) * GM_LDK + kk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      store_tile(lds[buf ^ 1][0], sa);
      store_tile(lds[buf ^ 1][1], sb);
    }
    __syncthreads();
    buf ^= 1;
  }

  // epilogue: lane holds column (lane&31) and rows 8*jj + 4*(lane>>5) + e
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t m = m0 + wm * 64 + i * 32 + jj * 8 + (lane >> 5) * 4 + e;
          if (m >= M) continue;
          const float v = alpha * acc[i][j][jj * 4 + e];
          if (EPI == ALODLM_EPI_STORE) {
            reinterpret_cast<bf16_t*>(C)[m * ldc + n] = float_to_bf16(v);
          } else if (EPI == ALODLM_EPI_RESIDUAL) {
            const float r = bf16_to_float(R[m * ldr + n]);
            reinterpret_cast<bf16_t*>(C)[m * ldc + n] = float_to_bf16(r + round_bf16(v));
          } else if (partial) {
            partial[((int64_t)blockIdx.y * M + m) * N + n] = v;
          } else {
            reinterpret_cast<float*>(C)[m * ldc + n] += v;
          }
        }
    }
}

// C[m, n] (+)= sum_s partial[s, m, n] (partials summed in split order, then
// added to C, or written over it when `overwrite`)
__global__ void splitk_reduce_kernel(const float* __restrict__ partial, int64_t splits, int64_t M,
                                     int64_t N, float* __restrict__ C, int64_t ldc,
                                     bool overwrite) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  float s = 0.f;
  for (int64_t p = 0; p < splits; ++p) s += partial[p * M * N + i];
  float* dst = C + (i / N) * ldc + (i % N);
  *dst = overwrite ? s : *dst + s;
}

// The same sum, 4 consecutive columns per thread (N, ldc multiples of 4, both
// buffers 16-byte aligned): grid.x covers a row's N/4 column groups, grid.y
// strides over rows, so no 64-bit division is needed.
__global__ void splitk_reduce4_kernel(const float* __restrict__ partial, int64_t splits,
                                      int64_t M, int64_t N, float* __restrict__ C, int64_t ldc,
                                      bool overwrite) {
  const int64_t n = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (n >= N) return;
  const int64_t plane = M * N;
  for (int64_t m = blockIdx.y; m < M; m += gridDim.y) {
    const float* src = partial + m * N + n;
    float4 s = *reinterpret_cast<const float4*>(src);
    for (int64_t p = 1; p < splits; ++p) {
      const float4 t = *reinterpret_cast<const float4*>(src + p * plane);
      s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
    }
    float4* dst = reinterpret_cast<float4*>(C + m * ldc + n);
    if (overwrite) {
      *dst = s;
    } else {
      float4 c = *dst;
      c.x += s.x; c.y += s.y; c.z += s.z; c.w += s.w;
      *dst = c;
    }
  }
}

// C[m, n] = bf16(sum_s partial[s, m, n]) (split order; the partials carry
// alpha): the STORE epilogue of a split product, rounded once.
__global__ void splitk_store_kernel(const float* __restrict__ partial, int64_t splits, int64_t M,
                                    int64_t N, bf16_t* __restrict__ C, int64_t ldc) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t plane = M * N;
  for (int64_t m = blockIdx.y; m < M; m += gridDim.y) {
    float s = partial[m * N + n];
    for (int64_t p = 1; p < splits; ++p) s += partial[p * plane + m * N + n];
    C[m * ldc + n] = float_to_bf16(s);
  }
}

static void splitk_store(const float* partial, int64_t splits, int64_t M, int64_t N, bf16_t* C,
                         int64_t ldc, hipStream_t st) {
  const dim3 grid(ceil_div_u(N, 256), (unsigned)(M < 65535 ? M : 65535));
  splitk_store_kernel<<<grid, 256, 0, st>>>(partial, splits, M, N, C, ldc);
}

static void splitk_reduce(const float* partial, int64_t splits, int64_t M, int64_t N, float* C,
                          int64_t ldc, hipStream_t st, bool overwrite = false) {
  const bool vec = N % 4 == 0 && ldc % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(partial) | reinterpret_cast<uintptr_t>(C)) & 15) == 0;
  if (vec) {
    const dim3 grid(ceil_div_u(N / 4, 256), (unsigned)(M < 65535 ? M : 65535));
    splitk_reduce4_kernel<<<grid, 256, 0, st>>>(partial, splits, M, N, C, ldc, overwrite);
  } else {
    splitk_reduce_kernel<<<ceil_div_u(M * N, 256), 256, 0, st>>>(partial, splits, M, N, C, ldc,
                                                                 overwrite);
  }
}

// C[m, n] = 0 for an [M, N] float matrix with row stride ldc (a fill kernel,
// not a memset, so that the launch can be captured in a graph).
__global__ void zero_rows_kernel(float* __restrict__ C, int64_t M, int64_t N, int64_t ldc) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  for (int64_t m = blockIdx.y; m < M; m += gridDim.y) C[m * ldc + n] = 0.f;
}

static void zero_rows(float* C, int64_t M, int64_t N, int64_t ldc, hipStream_t st) {
  const dim3 grid(ceil_div_u(N, 256), (unsigned)(M < 65535 ? M : 65535));
  zero_rows_kernel<<<grid, 256, 0, st>>>(C, M, N, ldc);
}

// ---------------------------------------------------------------------------
// Generic LDS-tiled FMA kernel (float, or any layout/shape).  64x64 tile,
// 256 threads with 4x4 outputs each, k-step 16.
// ---------------------------------------------------------------------------
template <typename T, int EPI>
__global__ void __launch_bounds__(256)
gemm_simple_kernel(const T* __restrict__ A, int64_t sam, int64_t sak, const T* __restrict__ B,
                   int64_t sbn, int64_t sbk, void* C, int64_t ldc, const T* R, int64_t ldr,
                   int64_t M, int64_t N, int64_t K, float alpha) {
  __shared__ float as[16][64 + 1], bs[16][64 + 1];
  const int64_t m0 = (int64_t)blockIdx.y * 64, n0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 16 * 64; e += 256) {
      const int kk = e / 64, rr = e % 64;
      const int64_t gk = k0 + kk;
      const int64_t gm = m0 + rr, gn = n0 + rr;
      as[kk][rr] = (gk < K && gm < M) ? Elem<T>::load(A, gm * sam + gk * sak) : 0.f;
      bs[kk][rr] = (gk < K && gn < N) ? Elem<T>::load(B, gn * sbn + gk * sbk) : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) { a[i] = as[kk][ty * 4 + i]; b[i] = bs[kk][tx * 4 + i]; }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += a[i] * b[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
      if (m >= M || n >= N) continue;
      const float v = alpha * acc[i][j];
      if (EPI == ALODLM_EPI_STORE) Elem<T>::store(reinterpret_cast<T*>(C), m * ldc + n, v);
      else if (EPI == ALODLM_EPI_RESIDUAL)
        Elem<T>::store(reinterpret_cast<T*>(C), m * ldc + n,
                       Elem<T>::load(R, m * ldr + n) + Elem<T>::round(v));
      else reinterpret_cast<float*>(C)[m * ldc + n] += v;
    }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
static bool mfma_eligible(const void* A, int64_t lda, int a_kmajor, const void* B, int64_t ldb,
                          int b_kmajor, int64_t M, int64_t N, int64_t K) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!al16(A) || !al16(B)) return false;
  // k-contiguous operands are staged in 8-element chunks along K; m/n-contiguous
  // ones guard every k row, so any K works for them
  if ((a_kmajor || b_kmajor) && K % 8 != 0) return false;
  if (lda % 8 != 0 || ldb % 8 != 0) return false;
  if (!a_kmajor && M % 4 != 0) return false;
  if (!b_kmajor && N % 4 != 0) return false;
  return true;
}

static int64_t splitk_count(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + GM_BM - 1) / GM_BM) * ((N + GM_BN - 1) / GM_BN);
  const int64_t ksteps = (K + GM_BK - 1) / GM_BK;
  int64_t splits = 1;
  while (tiles * splits < 1024 && ksteps / (splits * 2) >= 8) splits *= 2;
  return splits;
}

int64_t gemm_big_splits(int64_t M, int64_t N, int64_t K);
void gemm_big_launch(const bf16_t* A, int64_t lda, int a_kmajor, const bf16_t* B, int64_t ldb,
                     int b_kmajor, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                     int64_t N, int64_t K, float alpha, int epi, float* part, int64_t splits,
                     int64_t* nsplit_out, hipStream_t st);


// The 256x256 kernel takes the products whose output fills at least one tile.
// The 256x256 kernel needs whole 64-deep k tiles for k-contiguous operands.
static bool use_big(int64_t M, int64_t N, int64_t K, bool any_kmajor = false) {
  return M >= 256 && N >= 256 && K >= 64 && (!any_kmajor || K % 64 == 0);
}

extern "C" int64_t alodlm_gemm_workspace(int64_t M, int64_t N, int64_t K, int epilogue, int dtype) {
  if (dtype != ALODLM_BF16) return 0;
  if (epilogue == ALODLM_EPI_STORE) {
    const int64_t s = (M >= 256 && N >= 256 && K % 32 == 0) ? gemm_dl_store_splits(M, N, K) : 1;
    return s > 1 ? s * M * N : 0;
  }
  if (epilogue != ALODLM_EPI_ACCUM && epilogue != ALODLM_EPI_STORE_F32) return 0;
  int64_t s = splitk_count(M, N, K);
  if (use_big(M, N, K)) {
    const int64_t b = gemm_big_splits(M, N, K);
    s = b > s ? b : s;
  }
  if (M >= 256 && N >= 256 && K % 32 == 0) {
    const int64_t d = gemm_dl_splits(M, N, K);
    s = d > s ? d : s;
  }
  return s > 1 ? s * M * N : 0;
}

template <bool AK, bool BK>
static void launch_mfma(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                        int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N, int64_t K,
                        float alpha, int epi, float* workspace, int64_t splits, hipStream_t st) {
  const int64_t tiles = ((M + GM_BM - 1) / GM_BM) * ((N + GM_BN - 1) / GM_BN);
  int64_t kps = K;
  if (splits > 1) kps = (((K + splits - 1) / splits) + GM_BK - 1) / GM_BK * GM_BK;
  const int64_t nsplit = (K + kps - 1) / kps;
  dim3 grid((unsigned)tiles, (unsigned)nsplit);
  float* part = (epi == ALODLM_EPI_ACCUM && nsplit > 1) ? workspace : nullptr;
  if (epi == ALODLM_EPI_STORE)
    gemm_bf16_kernel<AK, BK, ALODLM_EPI_STORE><<<grid, GM_THREADS, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  else if (epi == ALODLM_EPI_RESIDUAL)
    gemm_bf16_kernel<AK, BK, ALODLM_EPI_RESIDUAL><<<grid, GM_THREADS, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  else
    gemm_bf16_kernel<AK, BK, ALODLM_EPI_ACCUM><<<grid, GM_THREADS, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  if (part) splitk_reduce(part, nsplit, M, N, (float*)C, ldc, st);
}

extern "C" int alodlm_gemm(const void* A, int64_t lda, int a_kmajor, const void* B, int64_t ldb,
                           int b_kmajor, void* C, int64_t ldc, const void* R, int64_t ldr,
                           int64_t M, int64_t N, int64_t K, float alpha, int epilogue, int dtype,
                           float* workspace, void* stream) {
  ALODLM_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "gemm: negative shape");
  ALODLM_CHECK_ARG(epilogue >= 0 && epilogue <= 3, "gemm: bad epilogue");
  ALODLM_CHECK_ARG(epilogue != ALODLM_EPI_RESIDUAL || R != nullptr, "gemm: residual needs R");
  if (M == 0 || N == 0) return ALODLM_OK;
  hipStream_t st = as_stream(stream);
  if (dtype == ALODLM_BF16 && mfma_eligible(A, lda, a_kmajor, B, ldb, b_kmajor, M, N, K) &&
      gemm_dl_eligible(lda, a_kmajor, ldb, b_kmajor, M, N, K)) {
    int64_t splits = 1;
    if (epilogue == ALODLM_EPI_ACCUM || epilogue == ALODLM_EPI_STORE_F32)
      splits = gemm_dl_splits(M, N, K);
    else if (epilogue == ALODLM_EPI_STORE) splits = gemm_dl_store_splits(M, N, K);
    if (splits > 1 && workspace == nullptr) splits = 1;
    if (splits > 1) {  // the launch splits K into chunks of whole 32-deep stages
      const int64_t kps = (((K + splits - 1) / splits) + 31) / 32 * 32;
      if ((K + kps - 1) / kps < 2) splits = 1;
    }
    // a split STORE product writes float partials (the ACCUM kernel with a
    // partial buffer), then one reduction rounds their sum to bf16
    const int launch_epi = (epilogue == ALODLM_EPI_STORE && splits > 1) ? ALODLM_EPI_ACCUM : epilogue;
    int64_t nsplit = 1;
    // an accumulated product's split 0 adds into C in its own epilogue, so the
    // reduction reads one partial plane fewer: C = (C + p0) + (p1 + ... )
    const int first_into_c = epilogue == ALODLM_EPI_ACCUM;
    gemm_dl_launch((const bf16_t*)A, lda, a_kmajor, (const bf16_t*)B, ldb, b_kmajor, C, ldc,
                   (const bf16_t*)R, ldr, M, N, K, alpha, launch_epi, workspace, splits, &nsplit,
                   first_into_c, st);
    ALODLM_CHECK_LAUNCH("gemm_bf16_dl");
    if ((launch_epi == ALODLM_EPI_ACCUM || launch_epi == ALODLM_EPI_STORE_F32) && nsplit > 1) {
      if (epilogue == ALODLM_EPI_STORE) splitk_store(workspace, nsplit, M, N, (bf16_t*)C, ldc, st);
      else if (first_into_c) splitk_reduce(workspace + M * N, nsplit - 1, M, N, (float*)C, ldc, st);
      else splitk_reduce(workspace, nsplit, M, N, (float*)C, ldc, st,
                         epilogue == ALODLM_EPI_STORE_F32);
      ALODLM_CHECK_LAUNCH("gemm_splitk_reduce");
    }
    return ALODLM_OK;
  }
  if (epilogue == ALODLM_EPI_STORE_F32) {
    // the other kernels accumulate into a zeroed output
    zero_rows((float*)C, M, N, ldc, st);
    ALODLM_CHECK_LAUNCH("gemm_zero_output");
    epilogue = ALODLM_EPI_ACCUM;
  }
  if (dtype == ALODLM_BF16 && mfma_eligible(A, lda, a_kmajor, B, ldb, b_kmajor, M, N, K) &&
      use_big(M, N, K, a_kmajor || b_kmajor)) {
    int64_t splits = 1;
    if (epilogue == ALODLM_EPI_ACCUM) {
      splits = gemm_big_splits(M, N, K);
      if (splits > 1 && workspace == nullptr) splits = 1;
    }
    int64_t nsplit = 1;
    gemm_big_launch((const bf16_t*)A, lda, a_kmajor, (const bf16_t*)B, ldb, b_kmajor, C, ldc,
                    (const bf16_t*)R, ldr, M, N, K, alpha, epilogue, workspace, splits, &nsplit, st);
    ALODLM_CHECK_LAUNCH("gemm_bf16_256");
    if (epilogue == ALODLM_EPI_ACCUM && nsplit > 1) {
      splitk_reduce(workspace, nsplit, M, N, (float*)C, ldc, st);
      ALODLM_CHECK_LAUNCH("gemm_splitk_reduce");
    }
    return ALODLM_OK;
  }
  if (dtype == ALODLM_BF16 && mfma_eligible(A, lda, a_kmajor, B, ldb, b_kmajor, M, N, K)) {
    int64_t splits = 1;
    if (epilogue == ALODLM_EPI_ACCUM) {
      splits = splitk_count(M, N, K);
      if (splits > 1 && workspace == nullptr) splits = 1;
    }
    const bf16_t* a = (const bf16_t*)A;
    const bf16_t* b = (const bf16_t*)B;
    const bf16_t* r = (const bf16_t*)R;
    if (a_kmajor && b_kmajor) launch_mfma<true, true>(a, lda, b, ldb, C, ldc, r, ldr, M, N, K, alpha, epilogue, workspace, splits, st);
    else if (a_kmajor) launch_mfma<true, false>(a, lda, b, ldb, C, ldc, r, ldr, M, N, K, alpha, epilogue, workspace, splits, st);
    else if (b_kmajor) launch_mfma<false, true>(a, lda, b, ldb, C, ldc, r, ldr, M, N, K, alpha, epilogue, workspace, splits, st);
    else launch_mfma<false, false>(a, lda, b, ldb, C, ldc, r, ldr, M, N, K, alpha, epilogue, workspace, splits, st);
    ALODLM_CHECK_LAUNCH("gemm_bf16");
    return ALODLM_OK;
  }
  const int64_t sam = a_kmajor ? lda : 1, sak = a_kmajor ? 1 : lda;
  const int64_t sbn = b_kmajor ? ldb : 1, sbk = b_kmajor ? 1 : ldb;
  dim3 grid(ceil_div_u(N, 64), ceil_div_u(M, 64));
  ALODLM_DISPATCH(dtype, T, {
    if (epilogue == ALODLM_EPI_STORE)
      gemm_simple_kernel<T, ALODLM_EPI_STORE><<<grid, 256, 0, st>>>(
          (const T*)A, sam, sak, (const T*)B, sbn, sbk, C, ldc, (const T*)R, ldr, M, N, K, alpha);
    else if (epilogue == ALODLM_EPI_RESIDUAL)
      gemm_simple_kernel<T, ALODLM_EPI_RESIDUAL><<<grid, 256, 0, st>>>(
          (const T*)A, sam, sak, (const T*)B, sbn, sbk, C, ldc, (const T*)R, ldr, M, N, K, alpha);
    else
      gemm_simple_kernel<T, ALODLM_EPI_ACCUM><<<grid, 256, 0, st>>>(
          (const T*)A, sam, sak, (const T*)B, sbn, sbk, C, ldc, (const T*)R, ldr, M, N, K, alpha);
  });
  ALODLM_CHECK_LAUNCH("gemm_simple");
  return ALODLM_OK;
}

extern "C" int alodlm_gemm_segk(const void* const* a_segs, const void* const* b_segs, int nseg,
                                int64_t seg_k, int64_t lda, int64_t ldb, void* C, int64_t ldc,
                                int64_t M, int64_t N, float alpha, int epilogue, float* workspace,
                                void* stream) {
  ALODLM_CHECK_ARG(nseg >= 1 && nseg <= KSEGS_MAX, "gemm_segk: 1 to 8 segments");
  ALODLM_CHECK_ARG(epilogue == ALODLM_EPI_ACCUM || epilogue == ALODLM_EPI_STORE_F32,
                   "gemm_segk: float32 output epilogues only");
  ALODLM_CHECK_ARG(M >= 0 && N >= 0 && seg_k > 0 && seg_k % 32 == 0,
                   "gemm_segk: segments must hold a positive multiple of 32 k rows");
  if (M == 0 || N == 0) return ALODLM_OK;
  const int64_t K = seg_k * nseg;
  ALODLM_CHECK_ARG(gemm_dl_eligible(lda, 0, ldb, 0, M, N, K),
                   "gemm_segk: M and N must be >= 256 and multiples of 8, lda/ldb multiples of 8");
  KSegs segs{};
  for (int i = 0; i < KSEGS_MAX; ++i) {
    const int s = i < nseg ? i : nseg - 1;
    ALODLM_CHECK_ARG(a_segs[s] != nullptr && b_segs[s] != nullptr, "gemm_segk: null segment");
    ALODLM_CHECK_ARG(mfma_eligible(a_segs[s], lda, 0, b_segs[s], ldb, 0, M, N, seg_k),
                     "gemm_segk: segment bases must be 16-byte aligned");
    segs.a[i] = (const bf16_t*)a_segs[s];
    segs.b[i] = (const bf16_t*)b_segs[s];
  }
  segs.k = seg_k;
  hipStream_t st = as_stream(stream);
  int64_t splits = gemm_dl_splits(M, N, K);
  if (splits > 1 && workspace == nullptr) splits = 1;
  if (splits > 1) {
    const int64_t kps = (((K + splits - 1) / splits) + 31) / 32 * 32;
    if ((K + kps - 1) / kps < 2) splits = 1;
  }
  const int first_into_c = epilogue == ALODLM_EPI_ACCUM;
  int64_t nsplit = 1;
  gemm_dl_launch(segs.a[0], lda, 0, segs.b[0], ldb, 0, C, ldc, nullptr, 0, M, N, K, alpha,
                 epilogue, workspace, splits, &nsplit, first_into_c, st, &segs);
  ALODLM_CHECK_LAUNCH("gemm_bf16_dl_segk");
  if (nsplit > 1) {
    if (first_into_c) splitk_reduce(workspace + M * N, nsplit - 1, M, N, (float*)C, ldc, st);
    else splitk_reduce(workspace, nsplit, M, N, (float*)C, ldc, st, true);
    ALODLM_CHECK_LAUNCH("gemm_splitk_reduce");
  }
  return ALODLM_OK;
}
