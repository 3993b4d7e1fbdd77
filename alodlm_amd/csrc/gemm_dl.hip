// bf16 GEMM with direct global->LDS staging for the large products of the
// step:  C[m, n] = alpha * sum_k A(m, k) B(n, k), operands k-contiguous or
// m/n-contiguous in any combination.
//
// 256x256 block tile, 32-deep k stages in a ring of STAGES LDS buffers.  Each
// stage is filled by global_load_lds_dwordx4 (lane i of an instruction
// writes the i-th 16-byte slot after the instruction's LDS base), issued
// STAGES-1 tiles ahead; there are no staging registers and no VALU copies.
// Loads address a wave-uniform tile origin plus a 32-bit lane offset; rows and
// columns past the operand's edge are clamped to its last valid row / chunk.
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
// Waves: 4 (2 x 2, 128x128 each, one per SIMD).  v_mfma_f32_32x32x16_bf16
// with the operands swapped (B rows as the MFMA's A operand), so each lane
// owns 4 consecutive output columns.  A 128x128 wave tile reads a third less
// LDS per MFMA than a 128x64 one; with one wave per SIMD the MFMA pipe is kept
// fed by an explicit per-k-step schedule: each of the 16 MFMAs of a k step is
// followed by one LDS fragment read of the next k step (first 8) or by the
// direct loads of a later stage (last 8), so no group of memory instructions
// ever stalls the MFMA issue.
//
// The step is power-bound on MI355X (the chip holds its 1400 W limit by
// lowering the clock), so the loop is shaped for energy per FLOP as much as
// for latency: fewer LDS bytes per MFMA and no redundant instructions.
//
// With one wave per SIMD every instruction of the loop takes an issue slot
// beside the MFMAs, so the loop carries no address arithmetic: the tile loop
// is unrolled over the STAGES stages of the ring, every fragment read is a
// per-lane base register plus an immediate (stage, k step and 32-row block
// are compile-time), every direct load sets M0 with one scalar add from a
// per-wave base, and the two tile origins advance by one 64-bit add per
// stage.  Per 32 MFMAs a stage issues 24 LDS reads, 8 direct loads and about
// 20 scalar instructions (84 with the addresses computed in the loop, which
// measured 3-8 % slower on every product of the step).
//
// Workgroup -> tile order: consecutive workgroups land on different XCDs, so
// the tile sequence is dealt out in contiguous chunks per XCD, then swept in
// groups of 3 tile rows (down a group, then across).
#include "common.h"
#include "lds_dma.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef short v4s_t __attribute__((ext_vector_type(4)));
#define LDS_AS __attribute__((address_space(3)))

namespace {

constexpr int TB = 256;              // block tile (m and n)
constexpr int KMIN = 32;             // k multiple every product must have

// One direct-load instruction: 16 bytes per lane from the wave-uniform tile
// origin `o` plus the lane's 32-bit offset, into the 16-byte slot lane of the
// LDS byte address m0v (wave-uniform).  M0 is an operand of the instruction,
// so the compiler sets it (one scalar add from a per-wave base) and knows its
// value; the load itself is not visible to the compiler (lds_dma.h).
__device__ __forceinline__ void dma16_m0(const char* o, uint32_t off, uint32_t m0v) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(o), "{m0}"(m0v) : "memory");
}

// Operand staging.  init() fixes this wave's lane offsets (relative to the
// tile origin, clamped so that rows / columns past the operand re-read its
// last valid row / chunk: they only feed outputs that are never stored) and
// the byte step from one k tile's origin to the next; init_frag() fixes the
// lane's fragment offsets within a stage, so that every fragment read is one
// base register plus an immediate (stage, k step and 32-row block are
// compile-time in the unrolled loop).  Instruction j of a stage is issued by
// wave j % NW into the 1024-byte slot j of the operand's stage.
template <bool KMAJ, int NW, int KD> struct Opnd;

// P[rows][ld], k contiguous: tile [256 rows][KD k], rows of 2*KD bytes
// (CH = KD/8 chunks), chunk' = chunk ^ f(row) with f(row) = (row / (16/CH)) % CH,
// so the 16 rows of a fragment read cover 16 distinct 4-bank groups.
template <int NW, int KD> struct Opnd<true, NW, KD> {
  static_assert(KD == 32 || KD == 64, "f(row) is invariant under +32 rows for these depths");
  static constexpr int CH = KD / 8, RB = 2 * KD, RPI = 1024 / RB;  // rows per instruction
  static constexpr int NINST = TB / RPI, PER = NINST / NW, OPB = TB * KD * 2;
  uint32_t off[PER];
  uint32_t fo[KD / 16];  // fragment offset of 32-row block 0, per k step
  int64_t ld, step;
  static __device__ __forceinline__ int f(int row) { return (row / (16 / CH)) % CH; }
  __device__ __forceinline__ void init(int64_t ld_, int64_t rows_left, int wave, int lane) {
    ld = ld_;
    step = 2 * KD;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = RPI * (wave + NW * i) + lane / CH;
      const int c = (lane % CH) ^ f(r);
      const int64_t rc = r < rows_left ? r : rows_left - 1;
      off[i] = (uint32_t)((rc * ld + 8 * c) * 2);
    }
  }
  // fragments of rows r0 + 32 * idx + lane % 32 (r0 a multiple of 32) of the
  // operand's stages, which start `region` bytes into the LDS array
  __device__ __forceinline__ void init_frag(int r0, int lane, int region) {
    const int row = r0 + (lane & 31), half = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < KD / 16; ++ks)
      fo[ks] = (uint32_t)(region + row * RB + (((2 * ks + half) ^ f(row)) << 4));
  }
  // tile origin: rows r0.., k from k0
  __device__ __forceinline__ const char* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return reinterpret_cast<const char*>(P + r0 * ld + k0);
  }
  // 32-row block idx, k step ks, from stage `stage` (lds: the LDS array)
  __device__ __forceinline__ bf16x8_t frag(const char* lds, int stage, int ks, int idx) const {
    return *reinterpret_cast<const bf16x8_t*>(lds + fo[ks] + (stage * OPB + idx * 32 * RB));
  }
};

// P[k][ld], m/n contiguous: tile [KD k][256], 512-byte rows, chunk' = chunk ^ 4*(k & 3).
template <int NW, int KD> struct Opnd<false, NW, KD> {
  static constexpr int NINST = KD / 2, PER = NINST / NW, OPB = TB * KD * 2;  // two k rows per instruction
  uint32_t off[PER];
  uint32_t fo[4];  // fragment offset of k step 0, per 32-column block
  int64_t ld, step;
  __device__ __forceinline__ void init(int64_t ld_, int64_t cols_left, int wave, int lane) {
    ld = ld_;
    step = 2 * KD * ld;
    const int last_chunk = (int)((cols_left < TB ? cols_left : TB) / 8) - 1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = wave + NW * i;
      const int row = 2 * j + (lane >> 5);  // k row of the stage
      int c = (lane & 31) ^ (4 * (row & 3));
      c = c < last_chunk ? c : last_chunk;
      off[i] = (uint32_t)((row * ld + 8 * c) * 2);
    }
  }
  // transposed fragments of columns r0 + 32 * idx + lane % 32 (r0 a multiple of
  // 32) of the operand's stages, which start `region` bytes into the LDS
  // array: per 16 lanes, two ds_read_b64_tr_b16 of k rows 8 half + {0..3} and
  // {4..7} (+ 16 ks)
  __device__ __forceinline__ void init_frag(int r0, int lane, int region) {
    const int s = lane & 15, g = (lane >> 4) & 1, half = lane >> 5;
#pragma unroll
    for (int idx = 0; idx < 4; ++idx) {
      const int c = (((r0 >> 5) + idx) * 4 + 2 * g + ((s & 3) >> 1)) ^ (4 * (s >> 2));
      fo[idx] = (uint32_t)(region + (8 * half + (s >> 2)) * 512 + c * 16 + (s & 1) * 8);
    }
  }
  __device__ __forceinline__ const char* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return reinterpret_cast<const char*>(P + k0 * ld + r0);
  }
  __device__ __forceinline__ bf16x8_t frag(const char* lds, int stage, int ks, int idx) const {
    const char* p0 = lds + fo[idx] + (stage * OPB + ks * 16 * 512);
    const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)p0);
    const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)(p0 + 4 * 512));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

}  // namespace

template <bool AK, bool BK, int EPI, int NW, int KD, int STAGES>
__global__ void __launch_bounds__(NW * 64, 1)
gemm_dl_kernel(const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ B,
               int64_t ldb, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
               int64_t N, int64_t K, float alpha, int64_t k_per_split, float* __restrict__ partial,
               int first_into_c) {
  static_assert(NW == 4, "the k-step schedule is written for 4 waves of 128x128");
  constexpr int WM = 128, WN = 128;
  constexpr int FI = WM / 32, FJ = WN / 32;
  constexpr int WAVES_N = TB / WN;
  constexpr int OPB = TB * KD * 2;   // bytes of one operand's stage
  constexpr int KS = KD / 16;         // k steps per stage
  // [operand][stage][OPB]: the A stages, then the B stages, so that every
  // fragment read is a base register plus an immediate below 64 KB
  __shared__ __attribute__((aligned(1024))) char lds[2][STAGES][OPB];

  const int tiles_m = (int)((M + TB - 1) / TB), tiles_n = (int)((N + TB - 1) / TB);
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;  // contiguous tile chunk per XCD
  // within a chunk, tiles go down groups of 3 tile rows, then across: an
  // XCD's 32 concurrent tiles share 3 A panels, which its L2 keeps for the
  // next tile columns (groups of 2, 3, 4, 8, 16, 32 rows measured on the
  // step's products: 2-3 best, 0.9 % of the 1.7B step over 8)
  const int group = 3, per_group = group * tiles_n;
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

  Opnd<AK, NW, KD> oa;
  Opnd<BK, NW, KD> ob;
  oa.init(lda, M - m0, wave, lane);
  ob.init(ldb, N - n0, wave, lane);
  oa.init_frag(wm * WM, lane, 0);
  ob.init_frag(wn * WN, lane, STAGES * OPB);
  (void)half;
  (void)col;

  f32x16_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Fragment registers: F[ks & 1] holds k step ks of the current tile.
  bf16x8_t fa[2][FI], fb[2][FJ];
  // Direct-load slots: MFMA slots 8..15 of every k step (of the k step after
  // the barrier too when the ring has 3+ stages: its target stage was freed
  // one barrier earlier); a stage's PL loads are spread evenly over them.
  constexpr int PA = Opnd<AK, NW, KD>::PER, PB = Opnd<BK, NW, KD>::PER, PL = PA + PB;
  constexpr int PRE = (KS - 1) * 8;                     // slots before the barrier
  constexpr int SLOTS = STAGES >= 3 ? KS * 8 : PRE;
  static_assert(PL <= SLOTS, "not enough direct-load slots");
  constexpr int DPRE = (PL * PRE + SLOTS - 1) / SLOTS;   // loads issued before the barrier
  // loads of this wave that may still be in flight at the barrier of tile tt
  // (tile tt+1 must have landed): whole later stages plus this tile's early ones
  constexpr int VM_LOOP = STAGES >= 3 ? (STAGES - 3) * PL + DPRE : 0;
  constexpr int VM_PRO = (STAGES - 2) * PL;

  // Origins of the next k tile to load (wave-uniform), advanced once per
  // stage.  Past the last tile they stay on it: its re-load goes to a stage
  // that is never read, which keeps the vmcnt waits uniform.
  const char* pa = oa.origin(A, m0, kbeg);
  const char* pb = ob.origin(B, n0, kbeg);
  int tl = 0;  // k tile at pa / pb
  auto advance = [&]() {
    if (tl + 1 < ntiles) {
      pa += oa.step;
      pb += ob.step;
    }
    ++tl;
  };
  // LDS byte address of this wave's first 1024-byte slot
  const uint32_t mw = lds_addr(lds) + (uint32_t)wave * 1024u;
  // load d of this wave's share of a stage: the tile at pa / pb into stage sl
  auto dma_one = [&](int sl, int d) {
    if (d < PA) dma16_m0(pa, oa.off[d], mw + (uint32_t)(sl * OPB + NW * d * 1024));
    else dma16_m0(pb, ob.off[d - PA], mw + (uint32_t)((STAGES + sl) * OPB + NW * (d - PA) * 1024));
  };
  const char* lds0 = lds[0][0];
  // fragment q of a k step, in the order the MFMAs consume them:
  // A0, B0, B1, B2, B3, A1, A2, A3
  auto read_one = [&](int set, int stage, int ks, int q) {
    const bool isa = q == 0 || q >= 5;
    const int idx = q == 0 ? 0 : (q >= 5 ? q - 4 : q - 1);
    if (isa) fa[set][idx] = oa.frag(lds0, stage, ks, idx);
    else fb[set][idx] = ob.frag(lds0, stage, ks, idx);
  };
  auto mma_one = [&](int set, int q) {
    const int i = q >> 2, j = q & 3;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[set][j], fa[set][i], acc[i][j], 0, 0, 0);
  };

  // Tile tt (in stage s = tt % STAGES): k steps 0 .. KS-2, then the barrier
  // that publishes tile tt+1 (this wave's loads of it are waited for first),
  // then k step KS-1, whose reads fetch tile tt+1's k step 0; the loads of
  // tile tt + STAGES - 1 go to the stage of tile tt - 1.  Every instruction
  // group is fenced with sched_barrier so the compiler keeps this order.  The
  // stage index is a compile-time constant in each unrolled copy.
  auto tile_body = [&](const int s) {
    const int sn = (s + 1) % STAGES, sl = (s + STAGES - 1) % STAGES;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks == KS - 1) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(VM_LOOP) : "memory");
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        mma_one(ks & 1, q);
        if (q < 8) {
          // after the last tile these reads fetch a stage that is never used
          if (ks + 1 < KS) read_one((ks + 1) & 1, s, ks + 1, q);
          else read_one(0, sn, 0, q);
        } else {
          const int slot = ks * 8 + (q - 8);
#pragma unroll
          for (int d = 0; d < PL; ++d)
            if ((d * SLOTS) / PL == slot) dma_one(sl, d);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    advance();
  };

  if (ntiles > 0) {  // (every split of an eligible product has k tiles)
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
#pragma unroll
      for (int d = 0; d < PL; ++d) dma_one(s, d);
      advance();
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(VM_PRO) : "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 8; ++q) read_one(0, 0, 0, q);
    for (int tt = 0; tt < ntiles;) {
#pragma unroll
      for (int s = 0; s < STAGES; ++s) {
        if (tt < ntiles) tile_body(s);
        ++tt;
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // bf16 outputs (STORE / RESIDUAL) go through LDS, so that global traffic is
  // whole 512-byte tile rows: the tile is written as bf16 into [256][256]
  // (chunk' = chunk ^ (row & 31)), then each thread moves 16-byte chunks, 32
  // threads per row (and reads the matching 16 bytes of R).
  bf16_t* Cb = reinterpret_cast<bf16_t*>(C);
  if constexpr (EPI == ALODLM_EPI_STORE || EPI == ALODLM_EPI_RESIDUAL) {
    const bool coalesced = ldc % 8 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0 &&
                           (EPI != ALODLM_EPI_RESIDUAL ||
                            (ldr % 8 == 0 && reinterpret_cast<uintptr_t>(R) % 16 == 0));
    if (coalesced) {
      char* tile = lds[0][0];  // 128 KB: the whole stage ring
      constexpr int ITER = TB * 32 / (NW * 64);
      const bool interior = m0 + TB <= M && n0 + TB <= N;
      // residual rows of an interior tile are fetched before the tile is
      // staged, so their latency overlaps the LDS writes
      uint4 rres[EPI == ALODLM_EPI_RESIDUAL ? ITER : 1];
      if constexpr (EPI == ALODLM_EPI_RESIDUAL) {
        if (interior) {
          const int64_t nr = n0 + (threadIdx.x & 31) * 8;
#pragma unroll
          for (int it = 0; it < ITER; ++it) {
            const int row = it * (NW * 64 / 32) + (int)(threadIdx.x >> 5);
            rres[it] = *reinterpret_cast<const uint4*>(R + (m0 + row) * ldr + nr);
          }
        }
      }
      // every wave is done with the stages (an LDS-only wait: the residual
      // loads above stay in flight)
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
      for (int i = 0; i < FI; ++i) {
        const int row = wm * WM + i * 32 + col;
#pragma unroll
        for (int j = 0; j < FJ; ++j)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int chunk = (wn * WN + j * 32) / 8 + jj;
            const f32x16_t& a = acc[i][j];
            *reinterpret_cast<uint2*>(tile + row * 512 + ((chunk ^ (row & 31)) << 4) + half * 8) =
                make_uint2(pack_bf16x2(alpha * a[jj * 4], alpha * a[jj * 4 + 1]),
                           pack_bf16x2(alpha * a[jj * 4 + 2], alpha * a[jj * 4 + 3]));
          }
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int chunk = threadIdx.x & 31;
      const int64_t n = n0 + chunk * 8;
      if (interior) {
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
          const int row = it * (NW * 64 / 32) + (int)(threadIdx.x >> 5);
          const uint4 w = *reinterpret_cast<const uint4*>(tile + row * 512 + ((chunk ^ (row & 31)) << 4));
          bf16_t* dst = Cb + (m0 + row) * ldc + n;
          if constexpr (EPI == ALODLM_EPI_RESIDUAL) {
            // reference order: x + round_bf16(proj), rounded once more
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
            const uint32_t rv[4] = {rres[it].x, rres[it].y, rres[it].z, rres[it].w};
            uint32_t ov[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float lo = bf16_to_float((bf16_t)(rv[e] & 0xffff)) + bf16_to_float((bf16_t)(wv[e] & 0xffff));
              const float hi = bf16_to_float((bf16_t)(rv[e] >> 16)) + bf16_to_float((bf16_t)(wv[e] >> 16));
              ov[e] = pack_bf16x2(lo, hi);
            }
            *reinterpret_cast<uint4*>(dst) = make_uint4(ov[0], ov[1], ov[2], ov[3]);
          } else {
            *reinterpret_cast<uint4*>(dst) = w;
          }
        }
        return;
      }
#pragma unroll 4
      for (int it = 0; it < TB * 32 / (NW * 64); ++it) {
        const int row = it * (NW * 64 / 32) + (int)(threadIdx.x >> 5);
        const int64_t m = m0 + row;
        if (m >= M || n >= N) continue;
        uint4 w = *reinterpret_cast<const uint4*>(tile + row * 512 + ((chunk ^ (row & 31)) << 4));
        if (EPI == ALODLM_EPI_RESIDUAL) {
          // reference order: x + round_bf16(proj), rounded once more
          float r[8], o[8];
          if (n + 8 <= N) {
            Vec8<bf16_t>::load(R + m * ldr + n, r);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = n + e < N ? bf16_to_float(R[m * ldr + n + e]) : 0.f;
          }
          const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            o[e] = r[e] + bf16_to_float((bf16_t)((e & 1) ? (wv[e >> 1] >> 16) : (wv[e >> 1] & 0xffff)));
          if (n + 8 <= N) {
            Vec8<bf16_t>::store(Cb + m * ldc + n, o);
            continue;
          }
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < N) Cb[m * ldc + n + e] = float_to_bf16(o[e]);
        } else {
          if (n + 8 <= N) {
            *reinterpret_cast<uint4*>(Cb + m * ldc + n) = w;
            continue;
          }
          const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < N) Cb[m * ldc + n + e] = (bf16_t)((e & 1) ? (wv[e >> 1] >> 16) : (wv[e >> 1] & 0xffff));
        }
      }
      return;
    }
  }

  // Direct epilogue (float outputs, and unaligned bf16 outputs): lane owns row
  // m = ... + col and columns n .. n+3 (n = 8*jj + 4*half).
  float* Cf = reinterpret_cast<float*>(C);
  // split 0 of an accumulated float product adds straight into C (the other
  // splits' partials are added by the reduction after this kernel)
  float* P = partial && !(first_into_c && blockIdx.y == 0)
                 ? partial + (int64_t)blockIdx.y * M * N : nullptr;
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
          } else if (EPI == ALODLM_EPI_STORE_F32) {
            *reinterpret_cast<float4*>(Cf + m * ldc + n) = make_float4(v[0], v[1], v[2], v[3]);
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
            else if (EPI == ALODLM_EPI_STORE_F32) Cf[m * ldc + n + e] = v[e];
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
  if (M < TB || N < TB || K < KMIN || K % KMIN != 0) return false;
  if (lda % 8 != 0 || ldb % 8 != 0) return false;
  if (!a_kmajor && M % 8 != 0) return false;
  if (!b_kmajor && N % 8 != 0) return false;
  return true;
}

// Splits of K for ALODLM_EPI_ACCUM products with few output tiles: the
// fewest (powers of two up to 8, each split keeping >= 32 k stages) whose
// rounds of 256 workgroups (one per CU) cost the least per unit of work.
// Splits that only add rounds cost float partials and their reduction: the
// 1.7B step's dW of the QKV and O projections take 2 and 4 splits (one
// round), 22 us faster each than at 4 and 8.
int64_t gemm_dl_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ((M + TB - 1) / TB) * ((N + TB - 1) / TB);
  const int64_t ksteps = K / KMIN;
  const int64_t cus = 256;
  auto cost = [&](int64_t s) { return (double)((tiles * s + cus - 1) / cus) / (double)s; };
  int64_t best = 1;
  for (int64_t s = 2; s <= 8 && ksteps / s >= 32; s *= 2)
    if (cost(s) < 0.98 * cost(best)) best = s;
  return best;
}

// Splits of a bf16-output (STORE) product: the fewest that bring the rounds
// of 256 workgroups (one per CU) within 8 % of the split-free work, so that a
// long-K product with few output tiles (the LM head's dX) does not leave CUs
// idle in its last round; only K >= 16384 (the partials' traffic is then
// small next to the product) and every split keeps >= 2048 of K.  1 when the
// tiles already fill the rounds.
int64_t gemm_dl_store_splits(int64_t M, int64_t N, int64_t K) {
  if (K < 16384) return 1;
  const int64_t tiles = ((M + TB - 1) / TB) * ((N + TB - 1) / TB);
  const int64_t cus = 256;
  auto cost = [&](int64_t s) { return (double)((tiles * s + cus - 1) / cus) / (double)s; };
  const double ideal = (double)tiles / (double)cus;
  if (cost(1) <= 1.08 * ideal) return 1;
  int64_t best = 1;
  for (int64_t s = 2; s <= 8 && K / s >= 2048; ++s)
    if (cost(s) < cost(best) && cost(best) - cost(s) > 0.02 * cost(1)) best = s;
  return best;
}

template <bool AK, bool BK, int NW, int KD, int ST>
static void launch_dl(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                      int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N, int64_t K,
                      float alpha, int epi, float* part, int64_t kps, int64_t nsplit,
                      int first_into_c, hipStream_t st) {
  const int64_t tiles = ((M + TB - 1) / TB) * ((N + TB - 1) / TB);
  dim3 grid((unsigned)tiles, (unsigned)nsplit);
  if (epi == ALODLM_EPI_STORE)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_STORE, NW, KD, ST><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
  else if (epi == ALODLM_EPI_RESIDUAL)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_RESIDUAL, NW, KD, ST><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
  else if (epi == ALODLM_EPI_STORE_F32 && part == nullptr)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_STORE_F32, NW, KD, ST><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
  else
    gemm_dl_kernel<AK, BK, ALODLM_EPI_ACCUM, NW, KD, ST><<<grid, NW * 64, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
}

template <bool AK, bool BK>
static void launch_layout(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                          int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N,
                          int64_t K, float alpha, int epi, float* part, int64_t kps,
                          int64_t nsplit, int first_into_c, hipStream_t st) {
  // 4 waves, 32-deep k stages in a ring of 4 (128 KB of LDS)
  launch_dl<AK, BK, 4, 32, 4>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, part, kps,
                              nsplit, first_into_c, st);
}

// Launch the direct-load kernel; `part` (splits*M*N floats) is used when
// splits > 1 (float-output epilogues only), the caller reduces it.  With
// `first_into_c` (an accumulated float product) split 0 adds its result into
// C itself and its partial plane is left unwritten: the caller then adds
// planes 1.. only.
void gemm_dl_launch(const bf16_t* A, int64_t lda, int a_kmajor, const bf16_t* B, int64_t ldb,
                    int b_kmajor, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                    int64_t N, int64_t K, float alpha, int epi, float* part, int64_t splits,
                    int64_t* nsplit_out, int first_into_c, hipStream_t st) {
  int64_t kps = K;
  if (splits > 1) kps = (((K + splits - 1) / splits) + KMIN - 1) / KMIN * KMIN;
  const int64_t nsplit = (K + kps - 1) / kps;
  *nsplit_out = nsplit;
  float* p = ((epi == ALODLM_EPI_ACCUM || epi == ALODLM_EPI_STORE_F32) && nsplit > 1) ? part : nullptr;
  if (a_kmajor && b_kmajor) launch_layout<true, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, st);
  else if (a_kmajor) launch_layout<true, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, st);
  else if (b_kmajor) launch_layout<false, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, st);
  else launch_layout<false, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, st);
}
