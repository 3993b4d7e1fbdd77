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
// before the current tile's MFMAs, as buffer loads from a descriptor re-based
// per k tile (scalar work) with lane offsets fixed for the whole kernel.
//
// Workgroup -> tile order: consecutive workgroups land on different XCDs, so
// the tile sequence is first dealt out in contiguous chunks per XCD (each XCD's
// L2 sees a compact block of C), then swept in groups of 8 tile rows.
#include "common.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

#define GB_TILE 256
#define GB_THREADS 256

// Buffer view of an operand from `base` to `end` (one past its last element):
// loads at or beyond `end` return zeros, so no load can leave the operand.
// Tiles are re-based every k step, which keeps every lane offset below 2^32.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gb_rsrc(const bf16_t* base, const bf16_t* end) {
  const int64_t bytes = (int64_t)(end - base) * 2;
  const int32_t nrec = bytes <= 0 ? 0 : (bytes >= 0xffffffffll ? -1 : (int32_t)(uint32_t)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, nrec, 0x00020000);
}

__device__ __forceinline__ uint4 gb_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint2 gb_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// k-contiguous operand P[rows][ld]: BKT/8 chunks of 8 k-values per thread.
// Rows past the operand read zeros or feed rows of C that are never stored.
// K must be a multiple of BKT (every k tile is whole).
template <int BKT> struct GbStageK {
  static constexpr int PER = BKT / 8;
  static constexpr int LOADS = PER, WRITES = PER, TRANSPOSES = 0;
  static constexpr int ROWS = GB_THREADS / (BKT / 8);  // rows per load round
  uint4 v[PER];
  uint32_t voff;
  int kc;
  __device__ __forceinline__ void init(int64_t ld) {
    const int row = threadIdx.x / (BKT / 8);
    kc = (threadIdx.x % (BKT / 8)) * 8;
    voff = (uint32_t)((row * ld + kc) * 2);
  }
  __device__ __forceinline__ void load(const bf16_t* P, int64_t ld, int64_t r0, const bf16_t* end,
                                       int64_t k0, int64_t kend) {
    (void)kend;
    const __amdgpu_buffer_rsrc_t rs = gb_rsrc(P + r0 * ld + k0, end);
    const uint32_t step = (uint32_t)(ROWS * ld * 2);
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = gb_load16(rs, voff + i * step);
  }
  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = threadIdx.x + GB_THREADS * i;
      const int row = c / (BKT / 8), kcc = (c % (BKT / 8)) * 8;
      *reinterpret_cast<uint4*>(lds + row * (BKT + 8) + kcc) = v[i];
    }
  }
};

// m/n-contiguous operand P[K][ld]: blocks of 8(k) x 4(m) per thread, transposed
// in registers.  Block b: the 16 lanes of a quarter-wave cover 4 row quads x 4
// k chunks, so their 16-byte LDS writes (row stride BKT + 8) hit distinct banks.
// k rows past the operand read zeros (buffer bound); m past the operand read
// values that only reach columns of C that are never stored.
template <int BKT> struct GbStageMN {
  static constexpr int PER = BKT / 32;
  static constexpr int LOADS = PER * 8, WRITES = PER * 4, TRANSPOSES = PER * 4;
  uint2 v[PER][8];
  static __device__ __forceinline__ void coords(int b, int& rq, int& kq) {
    const int rest = b >> 4;
    rq = (b & 3) + 4 * (rest & 15);
    kq = ((b >> 2) & 3) + 4 * (rest >> 4);
  }
  uint32_t voff[PER];
  __device__ __forceinline__ void init(int64_t ld) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int rq, kq;
      coords(threadIdx.x + GB_THREADS * i, rq, kq);
      voff[i] = (uint32_t)(((int64_t)kq * 8 * ld + rq * 4) * 2);
    }
  }
  __device__ __forceinline__ void load(const bf16_t* P, int64_t ld, int64_t r0, const bf16_t* end,
                                       int64_t k0, int64_t kend) {
    (void)kend;
    const __amdgpu_buffer_rsrc_t rs = gb_rsrc(P + k0 * ld + r0, end);
    const uint32_t row = (uint32_t)(ld * 2);
#pragma unroll
    for (int i = 0; i < PER; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[i][j] = gb_load8(rs, voff[i] + j * row);
  }
  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int rq, kq;
      coords(threadIdx.x + GB_THREADS * i, rq, kq);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // element r of k rows 2p and 2p+1: one v_perm_b32 per output word
        const uint32_t sel = (r & 1) ? 0x07060302u : 0x05040100u;
        uint32_t w[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint32_t a = (r < 2) ? v[i][2 * p].x : v[i][2 * p].y;
          const uint32_t c = (r < 2) ? v[i][2 * p + 1].x : v[i][2 * p + 1].y;
          w[p] = __builtin_amdgcn_perm(c, a, sel);
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

  // Tile coordinates in 32-bit scalar arithmetic (64-bit division would be
  // expanded on the vector unit, and everything derived from it - the buffer
  // descriptors included - would lose its uniformity).
  const int tiles_m = (int)((M + GB_TILE - 1) / GB_TILE), tiles_n = (int)((N + GB_TILE - 1) / GB_TILE);
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;  // contiguous tile chunk per XCD
  const int group = 8, per_group = group * tiles_n;
  const int g = t / per_group, first_m = g * group;
  const int gsize = (tiles_m - first_m) < group ? (tiles_m - first_m) : group;
  const int tm = first_m + (t % per_group) % gsize, tn = (t % per_group) / gsize;
  const int64_t m0 = __builtin_amdgcn_readfirstlane(tm * GB_TILE);
  const int64_t n0 = __builtin_amdgcn_readfirstlane(tn * GB_TILE);
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
  sa.init(lda);
  sb.init(ldb);
  // one past the last element of each operand
  const bf16_t* a_end = A + (AK ? (M - 1) * lda + K : (K - 1) * lda + M);
  const bf16_t* b_end = B + (BK ? (N - 1) * ldb + K : (K - 1) * ldb + N);
  // Prologue: tile 0 into LDS buffer 0, its first fragments into registers.
  const int ntiles = (int)((kend - kbeg + BKT - 1) / BKT);
  if (ntiles > 0) {
    sa.load(A, lda, m0, a_end, kbeg, kend);
    sb.load(B, ldb, n0, b_end, kbeg, kend);
    sa.store(lds[0][0]);
    sb.store(lds[0][1]);
  }
  __syncthreads();
  const int a_row = (wm * 128 + col) * LDT + half * 8, b_row = (wn * 128 + col) * LDT + half * 8;
  bf16x8_t fa[2][4], fb[2][4];
  auto read_frags = [&](int set, int buf, int ks) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fa[set][i] = *reinterpret_cast<const bf16x8_t*>(lds[buf][0] + a_row + i * 32 * LDT + ks);
      fb[set][i] = *reinterpret_cast<const bf16x8_t*>(lds[buf][1] + b_row + i * 32 * LDT + ks);
    }
  };
  // Operands swapped (B rows as the MFMA's A operand) so that the accumulator
  // rows run along n: each lane then owns 4 consecutive output columns.
  auto mfma16 = [&](int set) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[set][j], fa[set][i], acc[i][j], 0, 0, 0);
  };
  read_frags(0, 0, 0);

  // Main loop, one basic block per k tile (no branches, so the interleave
  // below holds): the next tile's global loads go out during k step 0 (a
  // zero-length buffer view on the last tile turns them into zeros), the
  // fragments of k step s+1 are read during the MFMAs of step s, and the next
  // tile is written to the other LDS buffer during step 3.  One barrier per
  // tile separates those writes from the reads of the next tile.
  static_assert(BKT == 64, "the interleave below assumes four 16-wide k steps");
  constexpr int NVMEM = GbStage<AK, BKT>::type::LOADS + GbStage<BK, BKT>::type::LOADS;
  constexpr int NWRITE = GbStage<AK, BKT>::type::WRITES + GbStage<BK, BKT>::type::WRITES;
  constexpr int NVALU_T = 4 * (GbStage<AK, BKT>::type::TRANSPOSES + GbStage<BK, BKT>::type::TRANSPOSES);
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    const int64_t kn = kbeg + (int64_t)(t + 1) * BKT;
    // k step 0: next tile's global loads, fragments of step 1
    __builtin_amdgcn_sched_barrier(0);
    sa.load(A, lda, m0, more ? a_end : A, kn, kend);
    sb.load(B, ldb, n0, more ? b_end : B, kn, kend);
    read_frags(1, buf, 16);
    mfma16(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);           // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           // DS read
      __builtin_amdgcn_sched_group_barrier(0x020, NVMEM / 8, 0);   // VMEM read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
    // k step 1
    read_frags(0, buf, 32);
    mfma16(1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
    // k step 2
    read_frags(1, buf, 48);
    mfma16(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
    // k step 3: next tile into the other LDS buffer
    sa.store(lds[buf ^ 1][0]);
    sb.store(lds[buf ^ 1][1]);
    mfma16(1);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NVALU_T / 16, 0);  // VALU (transposes)
      __builtin_amdgcn_sched_group_barrier(0x200, NWRITE / 16, 0);   // DS write
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    read_frags(0, buf ^ 1, 0);
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
                make_uint2(pack_bf16x2(v[0], v[1]),
                           pack_bf16x2(v[2], v[3]));
          } else if (EPI == ALODLM_EPI_RESIDUAL) {
            const uint2 r = *reinterpret_cast<const uint2*>(R + m * ldr + n);
            const float rv[4] = {bf16_to_float((bf16_t)(r.x & 0xffff)), bf16_to_float((bf16_t)(r.x >> 16)),
                                 bf16_to_float((bf16_t)(r.y & 0xffff)), bf16_to_float((bf16_t)(r.y >> 16))};
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = rv[e] + round_bf16(v[e]);
            *reinterpret_cast<uint2*>(Cb + m * ldc + n) =
                make_uint2(pack_bf16x2(o[0], o[1]),
                           pack_bf16x2(o[2], o[3]));
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
