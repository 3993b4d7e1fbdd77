// bf16 GEMM with direct global->LDS staging for the large products of the
// step:  C[m, n] = alpha * sum_k A(m, k) B(n, k), operands k-contiguous or
// m/n-contiguous in any combination.
//
// 256x256 block tile, 32-deep k stages in a ring of STAGES LDS buffers.  Each
// stage is filled by buffer_load_dwordx4 ... lds (lane i of an instruction
// writes the i-th 16-byte slot after the instruction's LDS base), issued
// STAGES-1 tiles ahead; there are no staging registers and no VALU copies.
// Buffer descriptors are re-based per tile, so lane offsets stay 32-bit and
// loads past the operand's end read zeros.
//
// LDS layouts (16-byte-chunk XOR swizzles, chosen by the source chunk of each
// direct-load lane):
//  * k-contiguous operand: [256 rows][32 k], 64-byte rows,
//    chunk' = chunk ^ ((row >> 2) & 3); a fragment read (16 consecutive rows,
//    one chunk each) touches 16 distinct 4-bank groups;
//  * m/n-contiguous operand: [32 k][256], 512-byte rows,
//    chunk' = chunk ^ 4*(k & 3); fragments come from ds_read_b64_tr_b16 (per
//    16 lanes: 4 k rows x 16 columns, result lane i = column i), and the 32
//    lanes of a read touch 4 rows x 4 chunks = 16 distinct 4-bank groups.
// Both give the MFMA operand "row i = lane % 32, k = 8*(lane / 32) + 0..7".
//
// Waves: NW = 8 (2 x 4, 128x64 each, two waves per SIMD) or NW = 4 (2 x 2,
// 128x128 each).  v_mfma_f32_32x32x16_bf16 with the operands swapped (B rows
// as the MFMA's A operand), so each lane owns 4 consecutive output columns.
//
// Workgroup -> tile order: consecutive workgroups land on different XCDs, so
// the tile sequence is dealt out in contiguous chunks per XCD, then swept in
// groups of 8 tile rows.
#include "common.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef short v4s_t __attribute__((ext_vector_type(4)));
#define LDS_AS __attribute__((address_space(3)))

namespace {

constexpr int TB = 256;              // block tile (m and n)
constexpr int KD = 32;               // k depth of a stage
constexpr int STAGES = 4;
constexpr int OPB = TB * KD * 2;     // bytes of one operand's stage (16 KB)
constexpr int NINST = OPB / 1024;    // direct-load instructions per operand and stage

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const bf16_t* base, const bf16_t* end) {
  const int64_t bytes = (int64_t)(end - base) * 2;
  const int32_t nrec = bytes <= 0 ? 0 : (bytes >= 0xffffffffll ? -1 : (int32_t)(uint32_t)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, nrec, 0x00020000);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LDS_AS void*)lds, 16, voff, 0, 0, 0);
}

// Operand staging.  init() fixes the lane offsets; issue() loads instructions
// j = first, first + step, ... of one stage; frag() reads one MFMA operand.
template <bool KMAJ> struct Opnd;

template <> struct Opnd<true> {  // P[rows][ld], k contiguous
  uint32_t voff;
  int64_t ld;
  __device__ __forceinline__ void init(int64_t ld_, int lane) {
    ld = ld_;
    const int c = (lane & 3) ^ ((lane >> 4) & 3);  // row 16j + lane/4: (row >> 2) & 3 = (lane >> 4) & 3
    voff = (uint32_t)(((lane >> 2) * ld + 8 * c) * 2);
  }
  // tile: rows r0.., k from k0
  __device__ __forceinline__ const bf16_t* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return P + r0 * ld + k0;
  }
  template <int NW>
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t r, char* stage, int wave) const {
#pragma unroll
    for (int i = 0; i < NINST / NW; ++i) {
      const int j = wave + NW * i;
      dma16(r, stage + j * 1024, voff + (uint32_t)(j * 32 * ld));
    }
  }
  // rows `row` (0..255) of the tile, k step ks (0..1), 8 k values at 8*half
  static __device__ __forceinline__ bf16x8_t frag(const char* stage, int row, int ks, int half, int lane) {
    (void)lane;
    const int c = (2 * ks + half) ^ ((row >> 2) & 3);
    return *reinterpret_cast<const bf16x8_t*>(stage + row * 64 + c * 16);
  }
};

template <> struct Opnd<false> {  // P[k][ld], m/n contiguous
  uint32_t voff[2];
  int64_t ld;
  __device__ __forceinline__ void init(int64_t ld_, int lane) {
    ld = ld_;
#pragma unroll
    for (int p = 0; p < 2; ++p) {  // instruction parity: rows 2j + lane/32
      const int row = 2 * p + (lane >> 5);
      const int c = (lane & 31) ^ (4 * (row & 3));
      voff[p] = (uint32_t)(((lane >> 5) * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ const bf16_t* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return P + k0 * ld + r0;
  }
  template <int NW>
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t r, char* stage, int wave) const {
#pragma unroll
    for (int i = 0; i < NINST / NW; ++i) {
      const int j = wave + NW * i;
      dma16(r, stage + j * 1024, voff[j & 1] + (uint32_t)(j * 4 * ld));
    }
  }
  // column `row` (0..255) of the tile, k step ks: two transposed reads of
  // k rows 16ks + 8half + {0..3} and {4..7}
  static __device__ __forceinline__ bf16x8_t frag(const char* stage, int row, int ks, int half, int lane) {
    const int s = lane & 15, g = (lane >> 4) & 1;
    const int kr = 16 * ks + 8 * half + (s >> 2);
    const int c = ((row >> 5) * 4 + 2 * g + ((s & 3) >> 1)) ^ (4 * (s >> 2));
    const char* p0 = stage + kr * 512 + c * 16 + (s & 1) * 8;
    const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)p0);
    const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)(p0 + 4 * 512));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

}  // namespace

#define GDL_WAIT_BARRIER(n) asm volatile("s_waitcnt vmcnt(" #n ")\n\ts_barrier" ::: "memory")

template <bool AK, bool BK, int EPI, int NW>
__global__ void __launch_bounds__(NW * 64, NW == 8 ? 2 : 1)
gemm_dl_kernel(const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ B,
               int64_t ldb, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
               int64_t N, int64_t K, float alpha, int64_t k_per_split, float* __restrict__ partial) {
  constexpr int WM = 128, WN = NW == 8 ? 64 : 128;
  constexpr int FI = WM / 32, FJ = WN / 32;
  constexpr int WAVES_N = TB / WN;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES][2][OPB];

  const int tiles_m = (int)((M + TB - 1) / TB), tiles_n = (int)((N + TB - 1) / TB);
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;  // contiguous tile chunk per XCD
  const int group = 8, per_group = group * tiles_n;
  const int g = t / per_group, first_m = g * group;
  const int gsize = (tiles_m - first_m) < group ? (tiles_m - first_m) : group;
  const int tm = first_m + (t % per_group) % gsize, tn = (t % per_group) / gsize;
  const int64_t m0 = __builtin_amdgcn_readfirstlane(tm * TB);
  const int64_t n0 = __builtin_amdgcn_readfirstlane(tn * TB);
  const int64_t kbeg = (int64_t)blockIdx.y * k_per_split;
  const int64_t kend = (kbeg + k_per_split) < K ? (kbeg + k_per_split) : K;
  const int ntiles = (int)((kend - kbeg + KD - 1) / KD);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int half = lane >> 5, col = lane & 31;

  Opnd<AK> oa;
  Opnd<BK> ob;
  oa.init(lda, lane);
  ob.init(ldb, lane);
  const bf16_t* a_end = A + (AK ? (M - 1) * lda + K : (K - 1) * lda + M);
  const bf16_t* b_end = B + (BK ? (N - 1) * ldb + K : (K - 1) * ldb + N);

  // Tile tt into stage tt % STAGES; tiles past the end load nothing (empty
  // buffer view) but still count in vmcnt, which keeps the waits uniform.
  auto issue = [&](int tt) {
    const bool live = tt < ntiles;
    const int64_t k0 = kbeg + (int64_t)tt * KD;
    char* st = lds[tt % STAGES][0];
    const bf16_t* ao = oa.origin(A, m0, k0);
    const bf16_t* bo = ob.origin(B, n0, k0);
    oa.template issue<NW>(rsrc(ao, live ? a_end : ao), st, wave);
    ob.template issue<NW>(rsrc(bo, live ? b_end : bo), st + OPB, wave);
  };

  f32x16_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment registers: F[0] holds k step 0 of the current tile, F[1] k step 1.
  bf16x8_t fa[2][FI], fb[2][FJ];
  auto read = [&](int set, int stage, int ks) {
    const char* sa = lds[stage][0];
    const char* sb = lds[stage][1];
#pragma unroll
    for (int i = 0; i < FI; ++i) fa[set][i] = Opnd<AK>::frag(sa, wm * WM + i * 32 + col, ks, half, lane);
#pragma unroll
    for (int j = 0; j < FJ; ++j) fb[set][j] = Opnd<BK>::frag(sb, wn * WN + j * 32 + col, ks, half, lane);
  };
  auto mma = [&](int set) {
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int j = 0; j < FJ; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[set][j], fa[set][i], acc[i][j], 0, 0, 0);
  };

  // Schedule per tile t (stage t % STAGES visible, F[0] = its k step 0):
  //   issue tile t + STAGES - 1 (into the stage of tile t - 1, fully read)
  //   read F[1] = k step 1;  MFMAs of F[0]
  //   wait for tile t + 1 and for F[1], barrier
  //   read F[0] = tile t + 1, k step 0;  MFMAs of F[1]
  // so every barrier has the MFMAs of one k step on each side of it.
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(s);
  if constexpr (NW == 8) GDL_WAIT_BARRIER(8);
  else GDL_WAIT_BARRIER(16);
  read(0, 0, 0);
  for (int tt = 0; tt < ntiles; ++tt) {
    const int stage = tt % STAGES;
    issue(tt + STAGES - 1);
    read(1, stage, 1);
    mma(0);
    // this wave's loads of tile tt + 1 are done once at most the later
    // STAGES - 2 tiles' loads are outstanding
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (NW == 8) GDL_WAIT_BARRIER(8);
    else GDL_WAIT_BARRIER(16);
    if (tt + 1 < ntiles) read(0, (tt + 1) % STAGES, 0);
    mma(1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // epilogue: lane owns row m = ... + col and columns n .. n+3 (n = 8*jj + 4*half)
  float* Cf = reinterpret_cast<float*>(C);
  bf16_t* Cb = reinterpret_cast<bf16_t*>(C);
  float* P = partial ? partial + (int64_t)blockIdx.y * M * N : nullptr;
  const int64_t ldo = P ? N : ldc;
  const bool vec = (ldo % 4 == 0) && (reinterpret_cast<uintptr_t>(P ? (void*)P : C) % 16 == 0) &&
                   (EPI != ALODLM_EPI_RESIDUAL ||
                    (ldr % 4 == 0 && reinterpret_cast<uintptr_t>(R) % 16 == 0));
#pragma unroll
  for (int i = 0; i < FI; ++i) {
    const int64_t m = m0 + wm * WM + i * 32 + col;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int64_t n = n0 + wn * WN + j * 32 + jj * 8 + half * 4;
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

// The direct-load kernel needs whole 32-deep k stages, 16-byte-aligned rows and,
// for m/n-contiguous operands, dimensions in whole 16-byte chunks.
bool gemm_dl_eligible(int64_t lda, int a_kmajor, int64_t ldb, int b_kmajor, int64_t M, int64_t N,
                      int64_t K) {
  if (M < TB || N < TB || K < KD || K % KD != 0) return false;
  if (lda % 8 != 0 || ldb % 8 != 0) return false;
  if (!a_kmajor && M % 8 != 0) return false;
  if (!b_kmajor && N % 8 != 0) return false;
  return true;
}

// Splits of K for ALODLM_EPI_ACCUM products with few output tiles.
int64_t gemm_dl_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + TB - 1) / TB) * ((N + TB - 1) / TB);
  const int64_t ksteps = K / KD;
  int64_t s = 1;
  while (tiles * s < 512 && ksteps / (s * 2) >= 32) s *= 2;
  return s;
}

template <bool AK, bool BK, int NW>
static void launch_dl(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                      int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N, int64_t K,
                      float alpha, int epi, float* part, int64_t kps, int64_t nsplit,
                      hipStream_t st) {
  const int64_t tiles = ((M + TB - 1) / TB) * ((N + TB - 1) / TB);
  dim3 grid((unsigned)tiles, (unsigned)nsplit);
  if (epi == ALODLM_EPI_STORE)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_STORE, NW><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  else if (epi == ALODLM_EPI_RESIDUAL)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_RESIDUAL, NW><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
  else
    gemm_dl_kernel<AK, BK, ALODLM_EPI_ACCUM, NW><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part);
}

#ifndef GEMM_DL_WAVES
#define GEMM_DL_WAVES 8
#endif

// Launch the direct-load kernel; `part` (splits*M*N floats) is used when
// splits > 1 (ALODLM_EPI_ACCUM only), the caller reduces it.
void gemm_dl_launch(const bf16_t* A, int64_t lda, int a_kmajor, const bf16_t* B, int64_t ldb,
                    int b_kmajor, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                    int64_t N, int64_t K, float alpha, int epi, float* part, int64_t splits,
                    int64_t* nsplit_out, hipStream_t st) {
  int64_t kps = K;
  if (splits > 1) kps = (((K + splits - 1) / splits) + KD - 1) / KD * KD;
  const int64_t nsplit = (K + kps - 1) / kps;
  *nsplit_out = nsplit;
  float* p = (epi == ALODLM_EPI_ACCUM && nsplit > 1) ? part : nullptr;
  constexpr int NW = GEMM_DL_WAVES;
  if (a_kmajor && b_kmajor) launch_dl<true, true, NW>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
  else if (a_kmajor) launch_dl<true, false, NW>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
  else if (b_kmajor) launch_dl<false, true, NW>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
  else launch_dl<false, false, NW>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, st);
}
