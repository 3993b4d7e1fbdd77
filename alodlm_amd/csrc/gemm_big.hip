// bf16 GEMM for the large products of the step (every layer GEMM at the
// 1.7B / 8B shapes and the LM head):  C[m, n] = alpha * sum_k A(m, k) B(n, k).
//
// 256x256 block tile, 4 wavefronts in a 2x2 grid, each owning a 128x128
// sub-tile held in 16 v_mfma_f32_32x32x16_bf16 accumulators (256 AGPRs).  Per
// 16-wide k step a wavefront reads 8 fragments from LDS for 16 MFMAs, which
// keeps LDS reads at half of the LDS bandwidth while the MFMA pipe is full.
// Tiles of A and B (BKT deep) are staged through double-buffered LDS rows
// padded by 8 elements; an m/n-contiguous operand is transposed on the way in
// by 8(k) x 4(m) register blocks.  The next k tile's global loads are issued
// before the current tile's MFMAs.
//
// Workgroup -> tile order: consecutive workgroups land on different XCDs, so
// the tile sequence is first dealt out in contiguous chunks per XCD (each XCD's
// L2 sees a compact block of C), then swept in groups of 8 tile rows.
#include "common.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

#define GB_TILE 256
#define GB_THREADS 256

template <int BKT> struct GbStageK {  // k-contiguous operand: BKT/8 chunks of 8 per thread
  static constexpr int PER = BKT / 8;
  uint4 v[PER];
  __device__ __forceinline__ void load(const bf16_t* P, int64_t ld, int64_t r0, int64_t rows,
                                       int64_t k0, int64_t K) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + GB_THREADS * i;
      const int row = c / (BKT / 8), kc = (c % (BKT / 8)) * 8;
      const int64_t gr = r0 + row, gk = k0 + kc;
      const bool ok = gr < rows && gk + 8 <= K;
      uint4 x = make_uint4(0, 0, 0, 0);
      if (ok) x = *reinterpret_cast<const uint4*>(P + gr * ld + gk);
      v[i] = x;
    }
  }
  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + GB_THREADS * i;
      const int row = c / (BKT / 8), kc = (c % (BKT / 8)) * 8;
      *reinterpret_cast<uint4*>(lds + row * (BKT + 8) + kc) = v[i];
    }
  }
};

template <int BKT> struct GbStageMN {  // m/n-contiguous operand: BKT/32 blocks of 8(k) x 4(m)
  static constexpr int PER = BKT / 32;
  uint2 v[PER][8];
  __device__ __forceinline__ void load(const bf16_t* P, int64_t ld, int64_t r0, int64_t rows,
                                       int64_t k0, int64_t K) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = threadIdx.x + GB_THREADS * i;
      const int rq = b % 64, kq = b / 64;
      const int64_t gr = r0 + rq * 4;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t gk = k0 + kq * 8 + j;
        uint2 x = make_uint2(0, 0);
        if (gk < K && gr + 4 <= rows) x = *reinterpret_cast<const uint2*>(P + gk * ld + gr);
        v[i][j] = x;
      }
    }
  }
  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = threadIdx.x + GB_THREADS * i;
      const int rq = b % 64, kq = b / 64;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t w[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t a = (r < 2) ? v[i][2 * p].x : v[i][2 * p].y;
          const uint32_t c = (r < 2) ? v[i][2 * p + 1].x : v[i][2 * p + 1].y;
          w[p] = (r & 1) ? ((a >> 16) | (c & 0xffff0000u)) : ((a & 0xffffu) | (c << 16));
        }
        *reinterpret_cast<uint4*>(lds + (rq * 4 + r) * (BKT + 8) + kq * 8) =
            make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
};

template <bool KM, int BKT> struct GbStage { typedef GbStageK<BKT> type; };
template <int BKT> struct GbStage<false, BKT> { typedef GbStageMN<BKT> type; };

template <bool AK, bool BK, int EPI, int BKT>
__global__ void __launch_bounds__(GB_THREADS, 1)
gemm_big_kernel(const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ B,
                int64_t ldb, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                int64_t N, int64_t K, float alpha, int64_t k_per_split, float* __restrict__ partial) {
  constexpr int LDT = BKT + 8;
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][2][GB_TILE * LDT];

  const int64_t tiles_m = (M + GB_TILE - 1) / GB_TILE, tiles_n = (N + GB_TILE - 1) / GB_TILE;
  const int64_t T = tiles_m * tiles_n;
  int64_t t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;  // contiguous tile chunk per XCD
  const int64_t group = 8, per_group = group * tiles_n;
  const int64_t g = t / per_group, first_m = g * group;
  const int64_t gsize = (tiles_m - first_m) < group ? (tiles_m - first_m) : group;
  const int64_t tm = first_m + (t % per_group) % gsize, tn = (t % per_group) / gsize;
  const int64_t m0 = tm * GB_TILE, n0 = tn * GB_TILE;
  const int64_t kbeg = (int64_t)blockIdx.y * k_per_split;
  const int64_t kend = (kbeg + k_per_split) < K ? (kbeg + k_per_split) : K;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, col = lane & 31;

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  typename GbStage<AK, BKT>::type sa;
  typename GbStage<BK, BKT>::type sb;
  int buf = 0;
  if (kbeg < kend) {
    sa.load(A, lda, m0, M, kbeg, kend);
    sb.load(B, ldb, n0, N, kbeg, kend);
    sa.store(lds[0][0]);
    sb.store(lds[0][1]);
  }
  __syncthreads();
  for (int64_t k0 = kbeg; k0 < kend; k0 += BKT) {
    const bool more = k0 + BKT < kend;
    if (more) {
      sa.load(A, lda, m0, M, k0 + BKT, kend);
      sb.load(B, ldb, n0, N, k0 + BKT, kend);
    }
    const bf16_t* la = lds[buf][0] + (wm * 128 + col) * LDT + half * 8;
    const bf16_t* lb = lds[buf][1] + (wn * 128 + col) * LDT + half * 8;
#pragma unroll
    for (int ks = 0; ks < BKT; ks += 16) {
      bf16x8_t fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        fa[i] = *reinterpret_cast<const bf16x8_t*>(la + i * 32 * LDT + ks);
        fb[i] = *reinterpret_cast<const bf16x8_t*>(lb + i * 32 * LDT + ks);
      }
    // Operands swapped (B rows as the MFMA's A operand) so that the accumulator
    // rows run along n: each lane then owns 4 consecutive output columns.
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
    }
    if (more) {
      sa.store(lds[buf ^ 1][0]);
      sb.store(lds[buf ^ 1][1]);
    }
    __syncthreads();
    buf ^= 1;
  }

  // epilogue: lane owns row m = ... + col and columns n .. n+3 (n = 8*jj + 4*half)
  float* Cf = reinterpret_cast<float*>(C);
  bf16_t* Cb = reinterpret_cast<bf16_t*>(C);
  float* P = partial ? partial + (int64_t)blockIdx.y * M * N : nullptr;
  const int64_t ldo = P ? N : ldc;
  // 4-wide stores need 4-aligned leading dimensions and 16-byte-aligned bases.
  const bool vec = (ldo % 4 == 0) && (reinterpret_cast<uintptr_t>(P ? (void*)P : C) % 16 == 0) &&
                   (EPI != ALODLM_EPI_RESIDUAL ||
                    (ldr % 4 == 0 && reinterpret_cast<uintptr_t>(R) % 16 == 0));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + wm * 128 + i * 32 + col;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int64_t n = n0 + wn * 128 + j * 32 + jj * 8 + half * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = alpha * acc[i][j][jj * 4 + e];
        if (vec && n + 4 <= N) {
          if (EPI == ALODLM_EPI_STORE) {
            *reinterpret_cast<uint2*>(Cb + m * ldc + n) =
                make_uint2((uint32_t)float_to_bf16(v[0]) | ((uint32_t)float_to_bf16(v[1]) << 16),
                           (uint32_t)float_to_bf16(v[2]) | ((uint32_t)float_to_bf16(v[3]) << 16));
          } else if (EPI == ALODLM_EPI_RESIDUAL) {
            const uint2 r = *reinterpret_cast<const uint2*>(R + m * ldr + n);
            const float rv[4] = {bf16_to_float((bf16_t)(r.x & 0xffff)), bf16_to_float((bf16_t)(r.x >> 16)),
                                 bf16_to_float((bf16_t)(r.y & 0xffff)), bf16_to_float((bf16_t)(r.y >> 16))};
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = rv[e] + round_bf16(v[e]);
            *reinterpret_cast<uint2*>(Cb + m * ldc + n) =
                make_uint2((uint32_t)float_to_bf16(o[0]) | ((uint32_t)float_to_bf16(o[1]) << 16),
                           (uint32_t)float_to_bf16(o[2]) | ((uint32_t)float_to_bf16(o[3]) << 16));
          } else if (P) {
            *reinterpret_cast<float4*>(P + m * N + n) = make_float4(v[0], v[1], v[2], v[3]);
          } else {
            float4* dst = reinterpret_cast<float4*>(Cf + m * ldc + n);
            float4 o = *dst;
            o.x += v[0]; o.y += v[1]; o.z += v[2]; o.w += v[3];
            *dst = o;
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (n + e >= N) continue;
            if (EPI == ALODLM_EPI_STORE) Cb[m * ldc + n + e] = float_to_bf16(v[e]);
            else if (EPI == ALODLM_EPI_RESIDUAL)
              Cb[m * ldc + n + e] = float_to_bf16(bf16_to_float(R[m * ldr + n + e]) + round_bf16(v[e]));
            else if (P) P[m * N + n + e] = v[e];
            else Cf[m * ldc + n + e] += v[e];
          }
        }
      }
  }
}

// Splits of K for ALODLM_EPI_ACCUM products with few output tiles.
int64_t gemm_big_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + GB_TILE - 1) / GB_TILE) * ((N + GB_TILE - 1) / GB_TILE);
  const int64_t ksteps = (K + 63) / 64;
  int64_t s = 1;
  while (tiles * s < 512 && ksteps / (s * 2) >= 16) s *= 2;
  return s;
}

template <bool AK, bool BK>
static void launch_big(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                       int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N, int64_t K,
                       float alpha, int epi, float* part, int64_t kps, int64_t nsplit,
                       hipStream_t st) {
  constexpr int BKT = 64;
  const int64_t tiles = ((M + GB_TILE - 1) / GB_TILE) * ((N + GB_TILE - 1) / GB_TILE);
  dim3 grid((unsigned)tiles, (unsigned)nsplit);
  if (epi == ALODLM_EPI_STORE)
    gemm_big_kernel<AK, BK, ALODLM_EPI_STORE, BKT><<<grid, GB_THREADS, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  else if (epi == ALODLM_EPI_RESIDUAL)
    gemm_big_kernel<AK, BK, ALODLM_EPI_RESIDUAL, BKT><<<grid, GB_THREADS, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  else
    gemm_big_kernel<AK, BK, ALODLM_EPI_ACCUM, BKT><<<grid, GB_THREADS, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
}

// Launch the 256x256 kernel; `part` (splits*M*N floats) is used when splits > 1
// (ALODLM_EPI_ACCUM only), the caller reduces it.
void gemm_big_launch(const bf16_t* A, int64_t lda, int a_kmajor, const bf16_t* B, int64_t ldb,
                     int b_kmajor, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                     int64_t N, int64_t K, float alpha, int epi, float* part, int64_t splits,
                     int64_t* nsplit_out, hipStream_t st) {
  int64_t kps = K;
  if (splits > 1) kps = (((K + splits - 1) / splits) + 63) / 64 * 64;
  const int64_t nsplit = (K + kps - 1) / kps;
  *nsplit_out = nsplit;
  float* p = (epi == ALODLM_EPI_ACCUM && nsplit > 1) ? part : nullptr;
  if (a_kmajor && b_kmajor) launch_big<true, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
  else if (a_kmajor) launch_big<true, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
  else if (b_kmajor) launch_big<false, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
  else launch_big<false, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
}
