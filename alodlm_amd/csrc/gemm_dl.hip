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
// Waves: 4 (2 x 2, 128x128 each, one per SIMD), v_mfma_f32_16x16x32_bf16 with
// the operands swapped (B rows as the MFMA's A operand), so each lane owns 4
// consecutive output columns of one row.  One 32-deep stage is one k step of
// 8 x 8 MFMAs per wave (256 accumulation registers).  The step is power-bound
// on MI355X (the chip holds its 1400 W limit by lowering the clock): with the
// same LDS bytes and direct loads, the 16x16x32 instruction runs the products
// at a 10-15 % higher clock than v_mfma_f32_32x32x16_bf16 (measured per
// kernel from GRBM_GUI_ACTIVE over its duration), which outweighs the few
// percent more cycles it takes; the 1.7B step ran 2.2 % faster with it.
//
// LDS layouts (16-byte-chunk XOR swizzles, chosen by the source chunk of each
// direct-load lane; measured free of bank conflicts for these fragment reads):
//  * k-contiguous operand: [256 rows][32 k], 64-byte rows,
//    chunk' = chunk ^ ((row >> 1) & 3); a fragment read takes rows
//    r + lane % 16, chunk lane / 16 (ds_read_b128);
//  * m/n-contiguous operand: [32 k][256], 512-byte rows,
//    chunk' = chunk ^ (4*(k & 3) ^ 2*((k >> 3) & 1)); fragments come from
//    ds_read_b64_tr_b16 (per 16 lanes: 4 k rows x 16 columns, result lane i =
//    column i), k rows 8 (lane / 16) + 0..3 and + 4..7.
// Both give the MFMA operand "row i = lane % 16, k = 8*(lane / 16) + 0..7".
//
// With one wave per SIMD every instruction of the loop takes an issue slot
// beside the MFMAs, and a 16x16x32 MFMA leaves room for about three: the loop
// carries no address arithmetic (the tile loop is unrolled over the STAGES
// stages of the ring, every fragment read is a per-lane base register plus an
// immediate, every direct load sets M0 with one scalar add from a per-wave
// base, the two tile origins advance by one 64-bit add per stage), and the
// memory instructions are spread one group per MFMA: with the 8 direct loads
// bunched into the first 8 MFMAs and 3 LDS reads after some, the same kernel
// ran 12 % slower.
//
// Workgroup -> tile order: consecutive workgroups land on different XCDs, so
// the tile sequence is dealt out in contiguous chunks per XCD, then swept in
// groups of 3 tile rows (down a group, then across).
#include "common.h"
#include "gemm_dl.h"
#include "lds_dma.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef short v4s_t __attribute__((ext_vector_type(4)));
#define LDS_AS __attribute__((address_space(3)))

namespace {

constexpr int TB = 256;              // block tile (m and n)
constexpr int KD = 32;               // k per stage
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
// base register plus an immediate (stage and 16-row block are compile-time in
// the unrolled loop).  Instruction j of a stage is issued by wave j % NW into
// the 1024-byte slot j of the operand's stage.
template <bool KMAJ, int NW> struct Opnd;

// P[rows][ld], k contiguous: tile [256 rows][32 k], 64-byte rows,
// chunk' = chunk ^ f(row), f(row) = (row / 2) % 4.  The fragment reads take 16
// rows per 16 lanes; the (row / 4) % 4 swizzle that suits 32-row fragments
// costs them about 4 bank-conflict cycles per read on MI355X.
template <int NW> struct Opnd<true, NW> {
  static constexpr int CH = KD / 8, RB = 2 * KD, RPI = 1024 / RB;  // rows per instruction
  static constexpr int NINST = TB / RPI, PER = NINST / NW, OPB = TB * KD * 2;
  uint32_t off[PER];
  uint32_t fo;  // fragment offset of 16-row block 0
  int64_t ld, step;
  static __device__ __forceinline__ int f(int row) { return (row >> 1) & 3; }
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
  // fragments of rows r0 + 16 * idx + lane % 16, 16-byte chunk lane / 16, of
  // the operand's stages, which start `region` bytes into the LDS array
  // (f(row) is invariant under +16 rows)
  __device__ __forceinline__ void init_frag(int r0, int lane, int region) {
    const int row = r0 + (lane & 15);
    fo = (uint32_t)(region + row * RB + (((lane >> 4) ^ f(row)) << 4));
  }
  // tile origin: rows r0.., k from k0
  __device__ __forceinline__ const char* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return reinterpret_cast<const char*>(P + r0 * ld + k0);
  }
  __device__ __forceinline__ bf16x8_t frag(const char* lds, int stage, int idx) const {
    return *reinterpret_cast<const bf16x8_t*>(lds + fo + (stage * OPB + idx * 16 * RB));
  }
};

// P[k][ld], m/n contiguous: tile [32 k][256], 512-byte rows, chunk' = chunk ^
// swz(k), swz(k) = 4*(k & 3) ^ 2*((k / 8) & 1).  A fragment read takes k rows
// 8 apart in one pass; without the second term they conflict.
template <int NW> struct Opnd<false, NW> {
  static constexpr int NINST = KD / 2, PER = NINST / NW, OPB = TB * KD * 2;  // two k rows per instruction
  uint32_t off[PER];
  uint32_t fo[4][2];
  int64_t ld, step;
  static __device__ __forceinline__ int swz(int k) { return 4 * (k & 3) ^ 2 * ((k >> 3) & 1); }
  __device__ __forceinline__ void init(int64_t ld_, int64_t cols_left, int wave, int lane) {
    ld = ld_;
    step = 2 * KD * ld;
    const int last_chunk = (int)((cols_left < TB ? cols_left : TB) / 8) - 1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = wave + NW * i;
      const int row = 2 * j + (lane >> 5);  // k row of the stage
      int c = (lane & 31) ^ swz(row);
      c = c < last_chunk ? c : last_chunk;
      off[i] = (uint32_t)((row * ld + 8 * c) * 2);
    }
  }
  // fragments of columns r0 + 16 * idx + lane % 16: per 16 lanes (g = lane /
  // 16), ds_read_b64_tr_b16 of k rows 8 g + {0..3} and 8 g + {4..7}.  Lane s of
  // a group reads k row s / 4, columns 8 ((s & 3) / 2) + 4 (s & 1) .. +3 of the
  // 16-column block.  With r0 a multiple of 128 the swizzle only permutes
  // chunks within 32-column blocks: block idx = 2 a + c reads at fo[a][c]
  // (source chunk 4 a + 2 c + b lands at 4 (a ^ m) + 2 (c ^ (g & 1)) + b).
  __device__ __forceinline__ void init_frag(int r0, int lane, int region) {
    const int s = lane & 15, g = lane >> 4, m = s >> 2, b = (s & 3) >> 1;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        fo[a][c] = (uint32_t)(region + (8 * g + m) * 512 +
                              ((r0 >> 3) + 4 * (a ^ m) + 2 * (c ^ (g & 1)) + b) * 16 + (s & 1) * 8);
  }
  __device__ __forceinline__ const char* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return reinterpret_cast<const char*>(P + k0 * ld + r0);
  }
  __device__ __forceinline__ bf16x8_t frag(const char* lds, int stage, int idx) const {
    const char* p0 = lds + fo[idx >> 1][idx & 1] + stage * OPB;
    const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)p0);
    const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)(p0 + 4 * 512));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};


// 64-deep stages (the two-stage ring of gemm_dl2_kernel).
template <bool KMAJ, int NW> struct Opnd64;

// P[rows][ld], k contiguous: a stage is 32 blocks of 1 KB, block b holding
// rows 8 b .. 8 b + 7 as [8 rows x k 0..31][8 rows x k 32..63] (64-byte rows,
// chunk' = chunk ^ f(row), f(row) = (row / 2) % 4): one direct-load
// instruction fills one block from 8 whole 128-byte row pieces, and the
// fragment reads keep 64-byte rows (measured free of bank conflicts).
template <int NW> struct Opnd64<true, NW> {
  static constexpr int NINST = TB / 8, PER = NINST / NW, OPB = TB * 64 * 2;
  uint32_t off[PER];
  uint32_t fo;
  int64_t ld, step;
  static __device__ __forceinline__ int f(int row) { return (row >> 1) & 3; }
  __device__ __forceinline__ void init(int64_t ld_, int64_t rows_left, int wave, int lane) {
    ld = ld_;
    step = 2 * 64;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int r = 8 * (wave + NW * i) + ((lane & 31) >> 2), h = lane >> 5;
      const int c = (lane & 3) ^ f(r);
      const int64_t rc = r < rows_left ? r : rows_left - 1;
      off[i] = (uint32_t)((rc * ld + 32 * h + 8 * c) * 2);
    }
  }
  // fragments of rows r0 + 16 idx + lane % 16, k step ks, chunk lane / 16
  __device__ __forceinline__ void init_frag(int r0, int lane, int region) {
    const int row = r0 + (lane & 15);
    fo = (uint32_t)(region + (row >> 3) * 1024 + (row & 7) * 64 + (((lane >> 4) ^ f(row)) << 4));
  }
  __device__ __forceinline__ const char* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return reinterpret_cast<const char*>(P + r0 * ld + k0);
  }
  __device__ __forceinline__ bf16x8_t frag(const char* lds, int stage, int ks, int idx) const {
    return *reinterpret_cast<const bf16x8_t*>(lds + fo + (stage * OPB + idx * 2048 + ks * 512));
  }
};

// P[k][ld], m/n contiguous: [64 k][256], 512-byte rows, chunk ^ swz(k) as in
// the 32-deep layout (k step ks reads k rows 32 ks + ..).
template <int NW> struct Opnd64<false, NW> {
  static constexpr int NINST = 64 / 2, PER = NINST / NW, OPB = TB * 64 * 2;
  uint32_t off[PER];
  uint32_t fo[4][2];
  int64_t ld, step;
  static __device__ __forceinline__ int swz(int k) { return 4 * (k & 3) ^ 2 * ((k >> 3) & 1); }
  __device__ __forceinline__ void init(int64_t ld_, int64_t cols_left, int wave, int lane) {
    ld = ld_;
    step = 2 * 64 * ld;
    const int last_chunk = (int)((cols_left < TB ? cols_left : TB) / 8) - 1;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int j = wave + NW * i;
      const int row = 2 * j + (lane >> 5);
      int c = (lane & 31) ^ swz(row);
      c = c < last_chunk ? c : last_chunk;
      off[i] = (uint32_t)((row * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ void init_frag(int r0, int lane, int region) {
    const int s = lane & 15, g = lane >> 4, m = s >> 2, b = (s & 3) >> 1;
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        fo[a][c] = (uint32_t)(region + (8 * g + m) * 512 +
                              ((r0 >> 3) + 4 * (a ^ m) + 2 * (c ^ (g & 1)) + b) * 16 + (s & 1) * 8);
  }
  __device__ __forceinline__ const char* origin(const bf16_t* P, int64_t r0, int64_t k0) const {
    return reinterpret_cast<const char*>(P + k0 * ld + r0);
  }
  __device__ __forceinline__ bf16x8_t frag(const char* lds, int stage, int ks, int idx) const {
    const char* p0 = lds + fo[idx >> 1][idx & 1] + stage * OPB + ks * 32 * 512;
    const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)p0);
    const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)(p0 + 4 * 512));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

}  // namespace

// Epilogue of a 256x256 output tile.  `quad(t, row, col, v)` gives this
// lane's t-th group of 4 outputs (t < 64): tile row, first of 4 consecutive
// tile columns and the unscaled sums (row and col are compile-time per t plus
// a per-lane part).  bf16 outputs (STORE / RESIDUAL) go through LDS (`tile`:
// TILE_LDS bytes, free once every wave has passed the loop), so that global
// traffic is whole 512-byte tile rows: the tile is written as bf16 into 256
// rows of TILE_ROW bytes (512 + 16 of padding, which keeps both the 8-byte
// writes of 16 rows and the 16-byte reads along a row free of bank conflicts
// with addresses that are a base plus an immediate), then each thread moves
// 16-byte chunks, 32 threads per row (and reads the matching 16 bytes of R).
// SCALE: multiply by alpha; the bf16-output kernels are instantiated with
// and without it (every product of the step has alpha = 1, and the 256
// multiplies per wave are a third of the epilogue's VALU work; one kernel
// holding both epilogues spilled registers).
constexpr int TILE_ROW = 528, TILE_LDS = TB * TILE_ROW;
template <int EPI, int NTHR, bool SCALE, typename Quad>
__device__ __forceinline__ void tile_epilogue(char* tile, Quad quad, void* C, int64_t ldc,
                                              const bf16_t* R, int64_t ldr, int64_t M, int64_t N,
                                              int64_t m0, int64_t n0, float alpha, float* partial,
                                              int first_into_c) {
  bf16_t* Cb = reinterpret_cast<bf16_t*>(C);
  if constexpr (EPI == ALODLM_EPI_STORE || EPI == ALODLM_EPI_RESIDUAL) {
    const bool coalesced = ldc % 8 == 0 && reinterpret_cast<uintptr_t>(C) % 16 == 0 &&
                           (EPI != ALODLM_EPI_RESIDUAL ||
                            (ldr % 8 == 0 && reinterpret_cast<uintptr_t>(R) % 16 == 0));
    if (coalesced) {
      constexpr int ITER = TB * 32 / NTHR;
      const bool interior = m0 + TB <= M && n0 + TB <= N;
      // residual rows of an interior tile are fetched before the tile is
      // staged, so their latency overlaps the LDS writes
      uint4 rres[EPI == ALODLM_EPI_RESIDUAL ? ITER : 1];
      if constexpr (EPI == ALODLM_EPI_RESIDUAL) {
        if (interior) {
          const int64_t nr = n0 + (threadIdx.x & 31) * 8;
#pragma unroll
          for (int it = 0; it < ITER; ++it) {
            const int row = it * (NTHR / 32) + (int)(threadIdx.x >> 5);
            rres[it] = *reinterpret_cast<const uint4*>(R + (m0 + row) * ldr + nr);
          }
        }
      }
      // every wave is done with the stages (an LDS-only wait: the residual
      // loads above stay in flight)
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
      for (int t = 0; t < 64; ++t) {
        int row, col;
        float v[4];
        quad(t, row, col, v);
        if (SCALE) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] *= alpha;
        }
        *reinterpret_cast<uint2*>(tile + row * TILE_ROW + col * 2) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      const int chunk = threadIdx.x & 31;
      const int64_t n = n0 + chunk * 8;
      if (interior) {
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
          const int row = it * (NTHR / 32) + (int)(threadIdx.x >> 5);
          const uint4 w = *reinterpret_cast<const uint4*>(tile + row * TILE_ROW + chunk * 16);
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
      for (int it = 0; it < ITER; ++it) {
        const int row = it * (NTHR / 32) + (int)(threadIdx.x >> 5);
        const int64_t m = m0 + row;
        if (m >= M || n >= N) continue;
        uint4 w = *reinterpret_cast<const uint4*>(tile + row * TILE_ROW + chunk * 16);
        const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
        if (EPI == ALODLM_EPI_RESIDUAL) {
          float r[8], o[8];
          if (n + 8 <= N) {
            Vec8<bf16_t>::load(R + m * ldr + n, r);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) r[e] = n + e < N ? bf16_to_float(R[m * ldr + n + e]) : 0.f;
          }
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
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (n + e < N) Cb[m * ldc + n + e] = (bf16_t)((e & 1) ? (wv[e >> 1] >> 16) : (wv[e >> 1] & 0xffff));
        }
      }
      return;
    }
  }

  // Direct epilogue (float outputs, and unaligned bf16 outputs): 4 consecutive
  // columns per quad.  Split 0 of an accumulated float product adds straight
  // into C (the other splits' partials are added by the reduction after this
  // kernel).
  float* Cf = reinterpret_cast<float*>(C);
  float* P = partial && !(first_into_c && blockIdx.y == 0)
                 ? partial + (int64_t)blockIdx.y * M * N : nullptr;
  const int64_t ldo = P ? N : ldc;
  const bool vec = (ldo % 4 == 0) && (reinterpret_cast<uintptr_t>(P ? (void*)P : C) % 16 == 0) &&
                   (EPI != ALODLM_EPI_RESIDUAL ||
                    (ldr % 4 == 0 && reinterpret_cast<uintptr_t>(R) % 16 == 0));
#pragma unroll
  for (int t = 0; t < 64; ++t) {
    int row, col;
    float v[4];
    quad(t, row, col, v);
    const int64_t m = m0 + row, n = n0 + col;
    if (m >= M) continue;
    if (SCALE) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] *= alpha;
    }
    if (vec && n + 4 <= N) {
      if (EPI == ALODLM_EPI_STORE) {
        *reinterpret_cast<uint2*>(Cb + m * ldc + n) =
            make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      } else if (EPI == ALODLM_EPI_RESIDUAL) {
        const uint2 r = *reinterpret_cast<const uint2*>(R + m * ldr + n);
        const float rv[4] = {bf16_to_float((bf16_t)(r.x & 0xffff)), bf16_to_float((bf16_t)(r.x >> 16)),
                             bf16_to_float((bf16_t)(r.y & 0xffff)), bf16_to_float((bf16_t)(r.y >> 16))};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = rv[e] + round_bf16(v[e]);
        *reinterpret_cast<uint2*>(Cb + m * ldc + n) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
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

// The kernel.  Each wave's 128x128 tile is 8 x 8 blocks of 16x16; the 64
// MFMAs of a stage are issued block column by block column (j outer).  Per
// tile tt (stage s):
//  * MFMAs 1, 5, 9, 17, 21, .., 33: the 8 direct loads of tile tt+STAGES-1
//    into the stage of tile tt-1 (freed by the previous barrier);
//  * after MFMA 7: wait for tile tt+1's loads, barrier (publishes tile tt+1;
//    every wave has finished reading tile tt);
//  * MFMAs 8..63: the fragments of tile tt+1.  B fragment j is reloaded in
//    place once its block column is done (at MFMA 8 (j+1)); the last one,
//    needed until MFMA 63, and the A fragments go to the other register set.
// Base of segment i (a select chain: no dynamic indexing of the argument).
__device__ __forceinline__ const bf16_t* seg_base(const bf16_t* const (&p)[KSEGS_MAX], int i) {
  const bf16_t* r = p[0];
#pragma unroll
  for (int j = 1; j < KSEGS_MAX; ++j) r = i == j ? p[j] : r;
  return r;
}

template <bool AK, bool BK, int EPI, int STAGES, bool SCALE, bool SEGK = false>
__global__ void __launch_bounds__(256, 1)
gemm_dl_kernel(const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ B,
               int64_t ldb, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
               int64_t N, int64_t K, float alpha, int64_t k_per_split, float* __restrict__ partial,
               int first_into_c, KSegs segs) {
  constexpr int NW = 4, WM = 128, WN = 128;
  constexpr int FI = WM / 16, FJ = WN / 16;
  constexpr int WAVES_N = TB / WN;
  constexpr int OPB = TB * KD * 2;
  static_assert(STAGES % 2 == 0 && STAGES >= 4, "fragment sets alternate with the stage parity");
  // the A stages, then the B stages; the output tile is staged over them
  constexpr int LDS_BYTES = 2 * STAGES * OPB > TILE_LDS ? 2 * STAGES * OPB : TILE_LDS;
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];

  const int tiles_m = (int)((M + TB - 1) / TB), tiles_n = (int)((N + TB - 1) / TB);
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;  // contiguous tile chunk per XCD
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

  Opnd<AK, NW> oa;
  Opnd<BK, NW> ob;
  oa.init(lda, M - m0, wave, lane);
  ob.init(ldb, N - n0, wave, lane);
  oa.init_frag(wm * WM, lane, 0);
  ob.init_frag(wn * WN, lane, STAGES * OPB);

  f32x4_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  bf16x8_t fa[2][FI], fb[FJ - 1], fbl[2];
  constexpr int PA = Opnd<AK, NW>::PER, PB = Opnd<BK, NW>::PER, PL = PA + PB;
  static_assert(PL <= 8, "load_slot places 8 direct loads per stage");
  // at the barrier of tile tt (after MFMA 7), tiles tt+2 .. tt+STAGES-2 and
  // the first loads of tile tt+STAGES-1 (issued after MFMAs 1 and 5) may be
  // in flight
  constexpr int VM_LOOP = (STAGES - 3) * PL + (PL < 2 ? PL : 2);
  constexpr int VM_PRO = (STAGES - 2) * PL;

  const bf16_t* A0 = A;
  const bf16_t* B0 = B;
  int64_t k0 = kbeg;
  int seg = 0, left = 0;  // segment of the next load and its tiles left (SEGK)
  if constexpr (SEGK) {
    seg = (int)(kbeg / segs.k);
    k0 = kbeg - (int64_t)seg * segs.k;
    A0 = seg_base(segs.a, seg);
    B0 = seg_base(segs.b, seg);
    left = (int)((segs.k - k0) / KD);
  }
  const char* pa = oa.origin(A0, m0, k0);
  const char* pb = ob.origin(B0, n0, k0);
  int tl = 0;
  auto advance = [&]() {
    if (tl + 1 < ntiles) {
      if constexpr (SEGK) {
        if (--left == 0) {  // the next tile opens the next segment
          ++seg;
          pa = oa.origin(seg_base(segs.a, seg), m0, 0);
          pb = ob.origin(seg_base(segs.b, seg), n0, 0);
          left = (int)(segs.k / KD);
        } else {
          pa += oa.step;
          pb += ob.step;
        }
      } else {
        pa += oa.step;
        pb += ob.step;
      }
    }
    ++tl;
  };
  const uint32_t mw = lds_addr(lds) + (uint32_t)wave * 1024u;
  auto dma_one = [&](int sl, int d) {
    if (d < PA) dma16_m0(pa, oa.off[d], mw + (uint32_t)(sl * OPB + NW * d * 1024));
    else dma16_m0(pb, ob.off[d - PA], mw + (uint32_t)((STAGES + sl) * OPB + NW * (d - PA) * 1024));
  };
  const char* lds0 = lds;

  // with one wave per SIMD a 16x16x32 MFMA leaves room for about three other
  // instructions, so the memory instructions are spread one group per MFMA.
  // The direct loads go out every 4 MFMAs from MFMA 1 (13, where the last B
  // fragment is read, skipped): their cost is not latency (never waiting for
  // them takes as long) but the vector-memory path and the LDS writes they
  // share with the fragment reads, and bunched into MFMAs 1..23 they ran 1-3 %
  // slower.
  auto load_slot = [](int q) {  // direct load issued after MFMA q, or -1
    if (q == 1 || q == 5) return q >> 2;                  // before the barrier
    if (q >= 9 && q <= 33 && (q & 3) == 1 && q != 13) return q < 13 ? 2 : (q - 9) / 4 + 1;
    return -1;
  };
  auto tile_body = [&](const int s) {
    const int sn = (s + 1) % STAGES, sl = (s + STAGES - 1) % STAGES;
    const int cur = s & 1, nxt = cur ^ 1;
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      const int i = q & 7, j = q >> 3, r = q & 7;
      if (j == FJ - 1)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fbl[cur], fa[cur][i], acc[i][j], 0, 0, 0);
      else
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[cur][i], acc[i][j], 0, 0, 0);
      const int d = load_slot(q);
      if (d >= 0 && d < PL) dma_one(sl, d);
      if (q == 7) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(VM_LOOP) : "memory");
      }
      // fragments of tile tt+1 (after the last tile they fetch a stage that is
      // never used): B block j-1 in place once its column is done, A block
      // j-1 two MFMAs later, the last B block and the last A block in between
      if (j >= 1) {
        if (r == 0) fb[j - 1] = ob.frag(lds0, sn, j - 1);
        if (r == 2 && j - 1 < FI - 1) fa[nxt][j - 1] = oa.frag(lds0, sn, j - 1);
        if (q == 13) fbl[nxt] = ob.frag(lds0, sn, FJ - 1);
        if (q == 60) fa[nxt][FI - 1] = oa.frag(lds0, sn, FI - 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    advance();
  };

  if (ntiles > 0) {
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) {
#pragma unroll
      for (int d = 0; d < PL; ++d) dma_one(s, d);
      advance();
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(VM_PRO) : "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FI; ++i) fa[0][i] = oa.frag(lds0, 0, i);
#pragma unroll
    for (int j = 0; j < FJ - 1; ++j) fb[j] = ob.frag(lds0, 0, j);
    fbl[0] = ob.frag(lds0, 0, FJ - 1);
    for (int tt = 0; tt < ntiles;) {
#pragma unroll
      for (int s = 0; s < STAGES; ++s) {
        if (tt < ntiles) tile_body(s);
        ++tt;
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // lane: output row 16 i + lane % 16 of the wave tile, columns
  // 16 j + 4 (lane / 16) .. +3
  auto quad = [&](int t, int& row, int& col, float* v) {
    const int i = t >> 3, j = t & 7;
    row = wm * WM + i * 16 + (lane & 15);
    col = wn * WN + j * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][e];
  };
  tile_epilogue<EPI, NW * 64, SCALE>(lds, quad, C, ldc, R, ldr, M, N, m0, n0, alpha, partial,
                              first_into_c);
}

// Two 64-deep stages (128 KB): one barrier per 128 MFMAs and 128-byte row
// pieces per direct load.  Per tile tt (stage s = tt % 2), k step 0 reads k
// step 1's fragments; after MFMA 7 of k step 1 the barrier publishes tile tt+1
// (all loads in flight are its) and frees stage s; the rest of k step 1 reads
// tile tt+1's k step 0 fragments and issues tile tt+2's loads into stage s.
template <bool AK, bool BK, int EPI, bool SCALE>
__global__ void __launch_bounds__(256, 1)
gemm_dl2_kernel(const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ B,
                int64_t ldb, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                int64_t N, int64_t K, float alpha, int64_t k_per_split, float* __restrict__ partial,
                int first_into_c) {
  constexpr int NW = 4, WM = 128, WN = 128, STAGES = 2, KD2 = 64;
  constexpr int FI = WM / 16, FJ = WN / 16;
  constexpr int WAVES_N = TB / WN;
  constexpr int OPB = TB * KD2 * 2;
  constexpr int LDS_BYTES = 2 * STAGES * OPB > TILE_LDS ? 2 * STAGES * OPB : TILE_LDS;
  __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];

  const int tiles_m = (int)((M + TB - 1) / TB), tiles_n = (int)((N + TB - 1) / TB);
  const int T = tiles_m * tiles_n;
  int t = blockIdx.x;
  if (T % 8 == 0) t = (t % 8) * (T / 8) + t / 8;
  const int group = 3, per_group = group * tiles_n;
  const int g = t / per_group, first_m = g * group;
  const int gsize = (tiles_m - first_m) < group ? (tiles_m - first_m) : group;
  const int tm = first_m + (t % per_group) % gsize, tn = (t % per_group) / gsize;
  const int64_t m0 = __builtin_amdgcn_readfirstlane(tm * TB);
  const int64_t n0 = __builtin_amdgcn_readfirstlane(tn * TB);
  const int64_t kbeg = (int64_t)blockIdx.y * k_per_split;
  const int64_t kend = (kbeg + k_per_split) < K ? (kbeg + k_per_split) : K;
  const int ntiles = (int)((kend - kbeg + KD2 - 1) / KD2);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  Opnd64<AK, NW> oa;
  Opnd64<BK, NW> ob;
  oa.init(lda, M - m0, wave, lane);
  ob.init(ldb, N - n0, wave, lane);
  oa.init_frag(wm * WM, lane, 0);
  ob.init_frag(wn * WN, lane, STAGES * OPB);

  f32x4_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i)
#pragma unroll
    for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  bf16x8_t fa[2][FI], fb[FJ - 1], fbl[2];
  constexpr int PA = Opnd64<AK, NW>::PER, PB = Opnd64<BK, NW>::PER, PL = PA + PB;
  static_assert(PL == 16, "load_slot places 16 direct loads per stage");

  const char* pa = oa.origin(A, m0, kbeg);
  const char* pb = ob.origin(B, n0, kbeg);
  int tl = 0;
  auto advance = [&]() {
    if (tl + 1 < ntiles) {
      pa += oa.step;
      pb += ob.step;
    }
    ++tl;
  };
  const uint32_t mw = lds_addr(lds) + (uint32_t)wave * 1024u;
  auto dma_one = [&](int sl, int d) {
    if (d < PA) dma16_m0(pa, oa.off[d], mw + (uint32_t)(sl * OPB + NW * d * 1024));
    else dma16_m0(pb, ob.off[d - PA], mw + (uint32_t)((STAGES + sl) * OPB + NW * (d - PA) * 1024));
  };
  const char* lds0 = lds;

  // direct loads after MFMA q of k step 1 (after the barrier), away from the
  // fragment-read slots (q % 8 == 0 or 2, 13, 60)
  auto load_slot = [](int q) {
    constexpr int slots[16] = {9, 11, 14, 17, 19, 22, 25, 27, 30, 33, 35, 38, 41, 43, 46, 49};
    for (int d = 0; d < 16; ++d)
      if (slots[d] == q) return d;
    return -1;
  };
  // one k step: 64 MFMAs on fragment set `cur`; the fragments of the next k
  // step (stage sr, k step kr) go to set `cur ^ 1`
  auto kstep = [&](const int cur, const int sr, const int kr, const bool last, const int s) {
    const int nxt = cur ^ 1;
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      const int i = q & 7, j = q >> 3, r = q & 7;
      if (j == FJ - 1)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fbl[cur], fa[cur][i], acc[i][j], 0, 0, 0);
      else
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fb[j], fa[cur][i], acc[i][j], 0, 0, 0);
      if (last) {
        if (q == 7) {
          __builtin_amdgcn_sched_barrier(0);
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        }
        const int d = load_slot(q);
        if (d >= 0) dma_one(s, d);
      }
      if (j >= 1) {
        if (r == 0) fb[j - 1] = ob.frag(lds0, sr, kr, j - 1);
        if (r == 2 && j - 1 < FI - 1) fa[nxt][j - 1] = oa.frag(lds0, sr, kr, j - 1);
        if (q == 13) fbl[nxt] = ob.frag(lds0, sr, kr, FJ - 1);
        if (q == 60) fa[nxt][FI - 1] = oa.frag(lds0, sr, kr, FI - 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto tile_body = [&](const int s) {
    kstep(0, s, 1, false, s);          // reads k step 1 of this tile
    kstep(1, s ^ 1, 0, true, s);       // barrier, reads k step 0 of tile tt+1, loads tile tt+2
    advance();
  };

  if (ntiles > 0) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
#pragma unroll
      for (int d = 0; d < PL; ++d) dma_one(s, d);
      advance();
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" :: "n"(PL) : "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < FI; ++i) fa[0][i] = oa.frag(lds0, 0, 0, i);
#pragma unroll
    for (int j = 0; j < FJ - 1; ++j) fb[j] = ob.frag(lds0, 0, 0, j);
    fbl[0] = ob.frag(lds0, 0, 0, FJ - 1);
    for (int tt = 0; tt < ntiles;) {
#pragma unroll
      for (int s = 0; s < STAGES; ++s) {
        if (tt < ntiles) tile_body(s);
        ++tt;
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  auto quad = [&](int t, int& row, int& col, float* v) {
    const int i = t >> 3, j = t & 7;
    row = wm * WM + i * 16 + (lane & 15);
    col = wn * WN + j * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][e];
  };
  tile_epilogue<EPI, NW * 64, SCALE>(lds, quad, C, ldc, R, ldr, M, N, m0, n0, alpha, partial,
                              first_into_c);
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

template <bool AK, bool BK, bool SCALE>
static void launch_scaled(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                          int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N,
                          int64_t K, float alpha, int epi, float* part, int64_t kps,
                          int64_t nsplit, int first_into_c, const KSegs* segs, hipStream_t st) {
  const int64_t tiles = ((M + TB - 1) / TB) * ((N + TB - 1) / TB);
  dim3 grid((unsigned)tiles, (unsigned)nsplit);
  // K over separate segments: the dW layout with float outputs only
  if constexpr (!AK && !BK && SCALE) {
    if (segs != nullptr) {
      if (epi == ALODLM_EPI_STORE_F32 && part == nullptr)
        gemm_dl_kernel<false, false, ALODLM_EPI_STORE_F32, 4, true, true><<<grid, 256, 0, st>>>(
            A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c, *segs);
      else
        gemm_dl_kernel<false, false, ALODLM_EPI_ACCUM, 4, true, true><<<grid, 256, 0, st>>>(
            A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c, *segs);
      return;
    }
  }
  // both operands k-contiguous: two 64-deep stages (128-byte row pieces per
  // direct load; 3-7 % faster than the 32-deep ring on every such product of
  // the step, and the same results: the k order of every sum is unchanged)
  if constexpr (AK && BK) {
    if (K % 64 == 0 && kps % 64 == 0) {
      if (epi == ALODLM_EPI_STORE)
        gemm_dl2_kernel<AK, BK, ALODLM_EPI_STORE, SCALE><<<grid, 256, 0, st>>>(
            A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
      else if (epi == ALODLM_EPI_RESIDUAL)  // (without the multiply it spills)
        gemm_dl2_kernel<AK, BK, ALODLM_EPI_RESIDUAL, true><<<grid, 256, 0, st>>>(
            A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
      else if constexpr (SCALE) {
        if (epi == ALODLM_EPI_STORE_F32 && part == nullptr)
          gemm_dl2_kernel<AK, BK, ALODLM_EPI_STORE_F32, true><<<grid, 256, 0, st>>>(
              A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
        else
          gemm_dl2_kernel<AK, BK, ALODLM_EPI_ACCUM, true><<<grid, 256, 0, st>>>(
              A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c);
      }
      return;
    }
  }
  // 4 waves, 32-deep k stages in a ring of 4 (128 KB of LDS)
  constexpr int ST = 4;
  if (epi == ALODLM_EPI_STORE)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_STORE, ST, SCALE><<<grid, 256, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c, KSegs{});
  else if (epi == ALODLM_EPI_RESIDUAL)
    gemm_dl_kernel<AK, BK, ALODLM_EPI_RESIDUAL, ST, SCALE><<<grid, 256, 0, st>>>(
        A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c, KSegs{});
  else if constexpr (SCALE) {
    if (epi == ALODLM_EPI_STORE_F32 && part == nullptr)
      gemm_dl_kernel<AK, BK, ALODLM_EPI_STORE_F32, ST, true><<<grid, 256, 0, st>>>(
          A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c, KSegs{});
    else
      gemm_dl_kernel<AK, BK, ALODLM_EPI_ACCUM, ST, true><<<grid, 256, 0, st>>>(
          A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, kps, part, first_into_c, KSegs{});
  }
}

template <bool AK, bool BK>
static void launch_layout(const bf16_t* A, int64_t lda, const bf16_t* B, int64_t ldb, void* C,
                          int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M, int64_t N,
                          int64_t K, float alpha, int epi, float* part, int64_t kps,
                          int64_t nsplit, int first_into_c, const KSegs* segs, hipStream_t st) {
  // the float-output epilogues keep the multiply: without it the compiler
  // hoists their loads of C and spills
  if (alpha == 1.f && (epi == ALODLM_EPI_STORE || epi == ALODLM_EPI_RESIDUAL))
    launch_scaled<AK, BK, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, part, kps,
                                 nsplit, first_into_c, segs, st);
  else
    launch_scaled<AK, BK, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, part, kps,
                                nsplit, first_into_c, segs, st);
}

// Launch the direct-load kernel; `part` (splits*M*N floats) is used when
// splits > 1 (float-output epilogues only), the caller reduces it.  With
// `first_into_c` (an accumulated float product) split 0 adds its result into
// C itself and its partial plane is left unwritten: the caller then adds
// planes 1.. only.
void gemm_dl_launch(const bf16_t* A, int64_t lda, int a_kmajor, const bf16_t* B, int64_t ldb,
                    int b_kmajor, void* C, int64_t ldc, const bf16_t* R, int64_t ldr, int64_t M,
                    int64_t N, int64_t K, float alpha, int epi, float* part, int64_t splits,
                    int64_t* nsplit_out, int first_into_c, hipStream_t st, const KSegs* segs) {
  int64_t kps = K;
  if (splits > 1) kps = (((K + splits - 1) / splits) + KMIN - 1) / KMIN * KMIN;
  const int64_t nsplit = (K + kps - 1) / kps;
  *nsplit_out = nsplit;
  float* p = ((epi == ALODLM_EPI_ACCUM || epi == ALODLM_EPI_STORE_F32) && nsplit > 1) ? part : nullptr;
  if (a_kmajor && b_kmajor) launch_layout<true, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, segs, st);
  else if (a_kmajor) launch_layout<true, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, segs, st);
  else if (b_kmajor) launch_layout<false, true>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, segs, st);
  else launch_layout<false, false>(A, lda, B, ldb, C, ldc, R, ldr, M, N, K, alpha, epi, p, kps, nsplit, first_into_c, segs, st);
}
