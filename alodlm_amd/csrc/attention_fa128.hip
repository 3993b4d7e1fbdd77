// bf16 flash attention for head_dim 128 on gfx950 (forward, dQ, dK/dV) under
// the dual-stream training mask (alodlm/batch.py:23-31, applied as in
// alodlm/model.py:65-73).
//
// LDS tiles are unpadded 256-byte rows with a 16-byte-chunk XOR swizzle,
//   physical chunk = chunk ^ swz(row),   swz(r) = 4*(r & 3) + ((r >> 2) & 3),
// chosen so that both access patterns are free of bank conflicts:
//  * a row fragment (16 consecutive rows, one chunk each) covers 16 distinct
//    chunks, i.e. all 64 banks once;
//  * a transposed fragment (ds_read_b64_tr_b16; 32 lanes read 4 consecutive
//    rows x 4 chunks) covers 16 distinct chunks as well.
// Tiles are filled by direct global->LDS loads (global_load_lds_dwordx4: lane
// i of a wavefront instruction writes the i-th 16-byte slot after the base;
// issued through lds_dma.h), so the swizzle is applied by the choice of source
// chunk and no register staging or VALU work is spent on copies.  Tiles are double-buffered: the
// next tile's loads are issued right after the barrier that publishes the
// current one and are complete (vmcnt) before the next barrier.
//
// ds_read_b64_tr_b16 within each 16-lane group: source lane s reads four
// consecutive bf16 X_s[0..3]; result lane i receives X_{4e + i/4}[i % 4] as
// its element e.  With source lane s pointing at row rb + s/4, columns
// c0 + 4*(s % 4), result lane i holds column c0 + i of rows rb..rb+3 - a
// fragment of the transposed tile, which is what the P.V, dS.K, P^T.dO and
// dS^T.Q products need as their A operand.
//
// Work split (four wavefronts per workgroup, two workgroups per CU):
//  * forward / dQ: a 128-row query tile of one head (32 rows per wavefront),
//    walking 64-key tiles with S^T = K.Q^T so each lane owns one query;
//  * dK/dV: a 128-key tile of one kv head (32 keys per wavefront; K fragments
//    in registers, the V tile in LDS), walking the query heads of its group and
//    the 32-row query tiles that see it, with S = Q.K^T so each lane owns one
//    key.
// The host lists tiles by decreasing in-stream start; forward and dQ take
// them in that order and dK/dV in reverse, so the heaviest tiles of each pass
// are dispatched first.
#include <type_traits>

#include "attention_common.h"
#include "lds_dma.h"

typedef short v4s_t __attribute__((ext_vector_type(4)));
#define LDS_AS __attribute__((address_space(3)))

namespace {

constexpr int HD = 128;     // head_dim
constexpr int ROWB = 256;   // bytes per LDS tile row
constexpr int KT = 64;      // keys per tile (forward / dQ)
constexpr int QT = 32;      // query rows per tile (dK/dV)

__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Stored dS (block size 32): the dK/dV pass writes dS^T in 32x32 blocks of
// one query head - [32 keys][32 queries] bf16, 64-byte key rows - for every
// (query tile, key tile) pair of 32-row tiles of a segment's streams that the
// mask allows:
//   clean query tile qt, clean key tile kt <= qt;
//   noisy query tile qt, clean key tile kt < qt, and noisy key tile qt.
// Blocks are numbered per segment, clean query tiles first (qt (qt + 1) / 2 +
// kt), then noisy ones (T (T + 1) / 2 + qt (qt + 1) / 2 + kt, with kt = qt for
// the noisy key tile), T = ceil(L / 32); ds_base[s] is the first block of
// segment s and block b of query head h sits at (h * ds_blocks + b) * 2 KB.
constexpr int DS_BLOCK_BYTES = 32 * 32 * 2;
constexpr int DS_RSRC_WORD3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int DS_NT = 2;                   // cache policy of the dS stores: nt
__device__ __forceinline__ int ds_half_blocks(int L) {
  const int T = (L + 31) / 32;
  return T * (T + 1) / 2;
}
__device__ __forceinline__ bool ds_allowed(bool qn, int qt, bool kn, int kt) {
  return kn ? (qn && kt == qt) : (qn ? kt < qt : kt <= qt);
}
__device__ __forceinline__ int ds_index(bool qn, int qt, bool kn, int kt, int half_blocks) {
  return (qn ? half_blocks : 0) + qt * (qt + 1) / 2 + (kn ? qt : kt);
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One wavefront instruction: tile rows [r0, r0 + 4) <- global rows
// min(g0 + r, gmax) of g (row stride ld elements).  r0 is wave-uniform.
__device__ __forceinline__ void dload4(char* tile, int r0, const bf16_t* g, int64_t ld, int64_t g0,
                                       int64_t gmax, int lane) {
  const int r = r0 + (lane >> 4);
  const int c = (lane & 15) ^ swz(r);
  int64_t gr = g0 + r;
  gr = gr < gmax ? gr : gmax;
  dma16_v(g + gr * ld + c * 8, lds_addr(tile + r0 * ROWB));
}

// A 64-key K/V tile pair (forward / dQ) by direct loads.  Load i of wavefront
// w fills tile rows x = 16 w + 4 i + lane / 16, 16-byte slot lane % 16, i.e.
// logical chunk (lane % 16) ^ swz(x) of the key's K / V row; the per-lane
// byte offsets of those chunks from the tile's first row are fixed for the
// whole walk (kv_lane_offsets), so a tile costs no vector arithmetic: the
// first rows' addresses are scalar pairs and the eight loads share one M0
// save.  l0 is the wavefront's first K row in the stage (its V rows follow
// KT rows later).  Every row of the tile must exist (first row + KT <= N).
struct KVLanes {
  uint32_t k[4], v[4];
};
__device__ __forceinline__ KVLanes kv_lane_offsets(int wave, int lane, int64_t ldk, int64_t ldv) {
  KVLanes o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int x = wave * 16 + 4 * i + (lane >> 4);
    const int c = (lane & 15) ^ swz(x);
    o.k[i] = (uint32_t)((x * ldk + c * 8) * 2);
    o.v[i] = (uint32_t)((x * ldv + c * 8) * 2);
  }
  return o;
}
__device__ __forceinline__ void issue_kv64(uint32_t l0, const bf16_t* kb, const bf16_t* vb,
                                           const KVLanes& o) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %[sv], m0\n\t"
      "s_mov_b32 m0, %[l0]\n\t"
      "global_load_lds_dwordx4 %[k0], %[kb]\n\t"
      "s_add_u32 m0, %[l0], %[r4]\n\t"
      "global_load_lds_dwordx4 %[k1], %[kb]\n\t"
      "s_add_u32 m0, %[l0], %[r8]\n\t"
      "global_load_lds_dwordx4 %[k2], %[kb]\n\t"
      "s_add_u32 m0, %[l0], %[r12]\n\t"
      "global_load_lds_dwordx4 %[k3], %[kb]\n\t"
      "s_add_u32 m0, %[l0], %[vr0]\n\t"
      "global_load_lds_dwordx4 %[v0], %[vb]\n\t"
      "s_add_u32 m0, %[l0], %[vr4]\n\t"
      "global_load_lds_dwordx4 %[v1], %[vb]\n\t"
      "s_add_u32 m0, %[l0], %[vr8]\n\t"
      "global_load_lds_dwordx4 %[v2], %[vb]\n\t"
      "s_add_u32 m0, %[l0], %[vr12]\n\t"
      "global_load_lds_dwordx4 %[v3], %[vb]\n\t"
      "s_mov_b32 m0, %[sv]"
      : [sv] "=&s"(saved)
      : [l0] "s"(l0), [kb] "s"(kb), [vb] "s"(vb), [k0] "v"(o.k[0]), [k1] "v"(o.k[1]),
        [k2] "v"(o.k[2]), [k3] "v"(o.k[3]), [v0] "v"(o.v[0]), [v1] "v"(o.v[1]),
        [v2] "v"(o.v[2]), [v3] "v"(o.v[3]), [r4] "n"(4 * ROWB), [r8] "n"(8 * ROWB),
        [r12] "n"(12 * ROWB), [vr0] "n"(KT * ROWB), [vr4] "n"((KT + 4) * ROWB),
        [vr8] "n"((KT + 8) * ROWB), [vr12] "n"((KT + 12) * ROWB)
      : "memory");
}

// A/B operand fragment from a row: 8 bf16 of chunk `chunk` of tile row `row`.
__device__ __forceinline__ bf16x8_t row_frag(const char* tile, int row, int chunk) {
  return *reinterpret_cast<const bf16x8_t*>(tile + row * ROWB + ((chunk ^ swz(row)) << 4));
}

// Operand fragment of the transposed tile: lane l holds column cb + l % 32 at
// rows rb..rb+3 (elements 0-3) and rb+8..rb+11 (elements 4-7), rb = r0 + 4*(l / 32)
// - the row order of an accumulator's elements [0, 8) read as the B operand.
__device__ __forceinline__ bf16x8_t tr_frag(const char* tile, int r0, int cb, int lane) {
  const int s = lane & 15, g = (lane >> 4) & 1, h = lane >> 5;
  const int row = r0 + 4 * h + (s >> 2);
  const int chunk = (cb >> 3) + 2 * g + ((s & 3) >> 1);
  const int sub = (s & 1) * 8;
  const char* p0 = tile + row * ROWB + ((chunk ^ swz(row)) << 4) + sub;
  const char* p1 = tile + (row + 8) * ROWB + ((chunk ^ swz(row + 8)) << 4) + sub;
  const v4s_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)p0);
  const v4s_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS_AS v4s_t*)p1);
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ f32x16_t mfma(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// acc += a * b with the accumulator held in AGPRs.  The register allocator
// otherwise moves long-lived accumulators between AGPRs and VGPRs around
// every use when the VGPRs are full.  gfx950 needs no wait states between
// MFMAs chained on one accumulator; a VALU read of `acc` needs 12 after the
// last such MFMA (mfma_acc_settle).
__device__ __forceinline__ void mfma_acc(f32x16_t& acc, bf16x8_t a, bf16x8_t b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_acc_settle() { asm volatile("s_nop 15" ::: "memory"); }
// A zero accumulator made in AGPRs (0 * 0 + 0), so that the register
// allocator keeps the accumulator's home there from the start.  The zero
// operand may have been written by the instruction just before: an MFMA
// reading a VGPR needs 2 wait states after a VALU write of it, which the
// compiler does not insert ahead of inline assembly.
__device__ __forceinline__ void mfma_acc_zero(f32x16_t& acc) {
  const bf16x8_t z = {0, 0, 0, 0, 0, 0, 0, 0};
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(acc) : "v"(z));
}

// d = a * b (d0: first k step, zero accumulator) / d += a * b with d in VGPRs
// for the VALU work that follows and b held in AGPRs.  A VALU read of d needs
// 12 wait states after the MFMA; callers place at least a block of other
// MFMAs in between, or mfma_acc_settle.
__device__ __forceinline__ void mfma_v0(f32x16_t& d, bf16x8_t a, bf16x8_t b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(d) : "v"(a), "a"(b));
}
__device__ __forceinline__ void mfma_v(f32x16_t& d, bf16x8_t a, bf16x8_t b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}

struct QTile {  // a 128-row query tile (forward / dQ)
  int64_t base;
  int L, start, q1, qi;
  bool valid;
};

__device__ __forceinline__ QTile query_tile(const int64_t* bounds, const int32_t* tiles, int t,
                                            int wave, int col) {
  QTile a;
  const int seg = tiles[2 * t];
  a.start = tiles[2 * t + 1];
  a.base = bounds[seg];
  a.L = (int)((bounds[seg + 1] - a.base) / 2);
  const int stream_end = a.start < a.L ? a.L : 2 * a.L;
  a.q1 = a.start + 128 < stream_end ? a.start + 128 : stream_end;
  a.qi = a.start + wave * 32 + col;
  a.valid = a.qi < a.q1;
  return a;
}

}  // namespace

// ---------------------------------------------------------------------------
// Forward: O = softmax(Q K^T * scale) V, lse per (head, row) in natural log.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256, 2)
fa128_fwd_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                 const bf16_t* __restrict__ v, int64_t ldv, const int64_t* __restrict__ bounds,
                 const int32_t* __restrict__ tiles, bf16_t* __restrict__ o,
                 float* __restrict__ lse, int64_t N, int nq, int nkv, int B, float scale) {
  __shared__ __attribute__((aligned(1024))) char lds[2][2][KT * ROWB];  // [stage][K | V]
  const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.x, hk = h / (nq / nkv);
  const QTile T = query_tile(bounds, tiles, blockIdx.y, wave, col);
  const int64_t base = T.base;
  const int L = T.L;
  const int64_t ldq = (int64_t)nq * HD, ldk = (int64_t)nkv * HD;
  const float c = scale * FA_LOG2E;

  bf16x8_t qf[HD / 16];
#pragma unroll
  for (int kk = 0; kk < HD / 16; ++kk) {
    if (T.valid) qf[kk] = load_frag(q + (base + T.qi) * ldq + h * HD + kk * 16 + half * 8);
    else qf[kk] = bf16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }
  f32x16_t oacc[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i) oacc[i] = zero16();
  float m = -INFINITY, l = 0.f;  // running maximum (log2 units) and sum

  const Interval2 mine = keys_of_query(T.qi, T.valid, L, B);
  const Interval2 R = key_ranges(T.start, T.q1, L, B);
  const Interval2 first = keys_of_query(T.start, true, L, B), last = keys_of_query(T.q1 - 1, true, L, B);
  const bf16_t* kh = k + hk * HD;
  const bf16_t* vh = v + hk * HD;
  const KVLanes kvo = kv_lane_offsets(wave, lane, ldk, ldv);
  const uint32_t lds_w = lds_addr(lds) + (uint32_t)(wave * 16 * ROWB);  // this wave's rows
  auto issue = [&](int stg, int k0) {
    const int64_t row0 = base + k0;
    if (row0 + KT <= N) {
      issue_kv64(lds_w + (uint32_t)(stg * (2 * KT * ROWB)), kh + row0 * ldk, vh + row0 * ldv, kvo);
    } else {  // keys past the pack's last row re-read it (they are masked)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r0 = wave * 16 + i * 4;
        dload4(lds[stg][0], r0, kh, ldk, row0, N - 1, lane);
        dload4(lds[stg][1], r0, vh, ldv, row0, N - 1, lane);
      }
    }
  };
  int r, k0;
  bool more = range_first(R, r, k0);
  // the register loads above are complete before any direct load is issued,
  // so the compiler has no reason to wait inside the loop
  __builtin_amdgcn_s_waitcnt(0);
  if (more) issue(0, k0);
  int stg = 0;
  while (more) {
    wait_vmem();
    __syncthreads();
    const int cur_k0 = k0;
    const int klo = r ? mine.lo1 : mine.lo0, khi = r ? mine.hi1 : mine.hi0;
    const bool full = cur_k0 >= (r ? last.lo1 : last.lo0) &&
                      cur_k0 + KT <= (r ? first.hi1 : first.hi0);
    more = range_next(R, KT, r, k0);
    if (more) issue(stg ^ 1, k0);
    const char* kt = lds[stg][0];
    const char* vt = lds[stg][1];
    f32x16_t sacc[2] = {zero16(), zero16()};
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        sacc[kb] = mfma(row_frag(kt, kb * 32 + col, kk * 2 + half), qf[kk], sacc[kb]);
    if (!full) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = cur_k0 + kb * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
          if (key < klo || key >= khi) sacc[kb][e] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, sacc[kb][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * c;
    if (__any(mx > m + FA_RESCALE)) {
      const bool raise = mx > m + FA_RESCALE;
      const float m_new = raise ? mx : m;
      const float corr = raise ? fast_exp2(m - m_new) : 1.f;  // 0 when m was -inf
      l *= corr;
#pragma unroll
      for (int i = 0; i < HD / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[i][e] *= corr;
      m = m_new;
    }
    const float m_use = m == -INFINITY ? 0.f : m;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = fast_exp2(fmaf(sacc[kb][e], c, -m_use));
        sacc[kb][e] = p;
        rs += p;
      }
    l += rs + __shfl_xor(rs, 32, 64);
#pragma unroll
    for (int st = 0; st < KT / 16; ++st) {
      const bf16x8_t pb = pack8(sacc[st >> 1], (st & 1) * 8);
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) oacc[db] = mfma(tr_frag(vt, st * 16, db * 32, lane), pb, oacc[db]);
    }
    stg ^= 1;
  }
  if (T.valid) {
    const float inv = 1.0f / l;
    bf16_t* orow = o + (base + T.qi) * ldq + h * HD;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + j * 8 + half * 4;
        *reinterpret_cast<uint2*>(orow + d) =
            make_uint2(pack2(oacc[db][j * 4] * inv, oacc[db][j * 4 + 1] * inv),
                       pack2(oacc[db][j * 4 + 2] * inv, oacc[db][j * 4 + 3] * inv));
      }
    if (half == 0) lse[(int64_t)h * N + base + T.qi] = m * FA_LN2 + logf(l);
  }
}

// ---------------------------------------------------------------------------
// dQ = scale * dS K,  dS = P * (dP - delta),  dP = dO V^T, with
// delta[h, r] = sum_e dO[r, h, e] * O[r, h, e] computed here from the dO
// fragments each lane already holds and written out for the dK/dV pass.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256, 2)
fa128_dq_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                const bf16_t* __restrict__ v, int64_t ldv, const float* __restrict__ lse,
                const bf16_t* __restrict__ o, float* __restrict__ delta,
                const bf16_t* __restrict__ dout, const int64_t* __restrict__ bounds,
                const int32_t* __restrict__ tiles, bf16_t* __restrict__ dq, int64_t N, int nq,
                int nkv, int B, float scale, int* __restrict__ counter) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *counter = 0;  // for dK/dV
  __shared__ __attribute__((aligned(1024))) char lds[2][2][KT * ROWB];  // [stage][K | V]
  const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.x, hk = h / (nq / nkv);
  const QTile T = query_tile(bounds, tiles, blockIdx.y, wave, col);
  const int64_t base = T.base;
  const int L = T.L;
  const int64_t ldq = (int64_t)nq * HD, ldk = (int64_t)nkv * HD;
  const float c = scale * FA_LOG2E;

  bf16x8_t qf[HD / 16], df[HD / 16];
#pragma unroll
  for (int kk = 0; kk < HD / 16; ++kk) {
    if (T.valid) {
      qf[kk] = load_frag(q + (base + T.qi) * ldq + h * HD + kk * 16 + half * 8);
      df[kk] = load_frag(dout + (base + T.qi) * ldq + h * HD + kk * 16 + half * 8);
    } else {
      qf[kk] = bf16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      df[kk] = qf[kk];
    }
  }
  const float lse2 = T.valid ? lse[(int64_t)h * N + base + T.qi] * FA_LOG2E : 0.f;
  // delta of this lane's query: its 64 head_dim values, then the other half's
  float delta_q = 0.f;
  if (T.valid) {
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      const bf16x8_t of = load_frag(o + (base + T.qi) * ldq + h * HD + kk * 16 + half * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        delta_q += bf16_to_float((bf16_t)df[kk][e]) * bf16_to_float((bf16_t)of[e]);
    }
  }
  delta_q += __shfl_xor(delta_q, 32, 64);
  if (T.valid && half == 0) {
    delta[(int64_t)h * N + base + T.qi] = delta_q;
    delta[(int64_t)(nq + h) * N + base + T.qi] = lse2;  // lse * log2(e) for the dK/dV pass
  }
  f32x16_t acc[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i) acc[i] = zero16();

  const Interval2 mine = keys_of_query(T.qi, T.valid, L, B);
  const Interval2 R = key_ranges(T.start, T.q1, L, B);
  const Interval2 first = keys_of_query(T.start, true, L, B), last = keys_of_query(T.q1 - 1, true, L, B);
  const bf16_t* kh = k + hk * HD;
  const bf16_t* vh = v + hk * HD;
  const KVLanes kvo = kv_lane_offsets(wave, lane, ldk, ldv);
  const uint32_t lds_w = lds_addr(lds) + (uint32_t)(wave * 16 * ROWB);  // this wave's rows
  auto issue = [&](int stg, int k0) {
    const int64_t row0 = base + k0;
    if (row0 + KT <= N) {
      issue_kv64(lds_w + (uint32_t)(stg * (2 * KT * ROWB)), kh + row0 * ldk, vh + row0 * ldv, kvo);
    } else {  // keys past the pack's last row re-read it (they are masked)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r0 = wave * 16 + i * 4;
        dload4(lds[stg][0], r0, kh, ldk, row0, N - 1, lane);
        dload4(lds[stg][1], r0, vh, ldv, row0, N - 1, lane);
      }
    }
  };
  int r, k0;
  bool more = range_first(R, r, k0);
  // the register loads above are complete before any direct load is issued,
  // so the compiler has no reason to wait inside the loop
  __builtin_amdgcn_s_waitcnt(0);
  if (more) issue(0, k0);
  int stg = 0;
  while (more) {
    wait_vmem();
    __syncthreads();
    const int cur_k0 = k0;
    const int klo = r ? mine.lo1 : mine.lo0, khi = r ? mine.hi1 : mine.hi0;
    const bool full = cur_k0 >= (r ? last.lo1 : last.lo0) &&
                      cur_k0 + KT <= (r ? first.hi1 : first.hi0);
    more = range_next(R, KT, r, k0);
    if (more) issue(stg ^ 1, k0);
    const char* kt = lds[stg][0];
    const char* vt = lds[stg][1];
    f32x16_t sacc[2] = {zero16(), zero16()}, pacc[2] = {zero16(), zero16()};
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = mfma(row_frag(kt, kb * 32 + col, kk * 2 + half), qf[kk], sacc[kb]);
        pacc[kb] = mfma(row_frag(vt, kb * 32 + col, kk * 2 + half), df[kk], pacc[kb]);
      }
    // dS^T = P^T * (dP^T - delta), P^T = exp(S^T * scale - lse)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float p = fast_exp2(fmaf(sacc[kb][e], c, -lse2));
        if (!full) {
          const int key = cur_k0 + kb * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
          if (key < klo || key >= khi) p = 0.f;
        }
        sacc[kb][e] = p * (pacc[kb][e] - delta_q);
      }
#pragma unroll
    for (int st = 0; st < KT / 16; ++st) {
      const bf16x8_t ds = pack8(sacc[st >> 1], (st & 1) * 8);
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) acc[db] = mfma(tr_frag(kt, st * 16, db * 32, lane), ds, acc[db]);
    }
    stg ^= 1;
  }
  if (T.valid) {
    bf16_t* row = dq + (base + T.qi) * ldq + h * HD;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + j * 8 + half * 4;
        *reinterpret_cast<uint2*>(row + d) =
            make_uint2(pack2(acc[db][j * 4] * scale, acc[db][j * 4 + 1] * scale),
                       pack2(acc[db][j * 4 + 2] * scale, acc[db][j * 4 + 3] * scale));
      }
  }
}

// ---------------------------------------------------------------------------
// dV = P^T dO,  dK = scale * dS^T Q.  lse2[h, r] = lse[h, r] * log2(e), as the
// dQ pass writes it next to delta.
//
// One wavefront per SIMD (one workgroup per CU, so each lane may hold up to
// 512 registers).  K and V of the wavefront's 32 keys stay in registers as B
// operands.  Query tiles (32 rows of Q and dO with their lse2 and delta)
// stream through a ring of DK_STAGES LDS stages.  The loop is
// software-pipelined; iteration i runs:
//   A  S and dP of tile i+1 (16 MFMAs), with the VALU work of tile i (P, dS,
//      bf16 packing) placed between them;
//   -  a barrier: tile i+2 has landed and the stage of tile i-1 is free;
//   -  the direct loads of tile i + DK_STAGES - 1 into that stage;
//   B  dV and dK of tile i (16 MFMAs), with the LDS reads of tile i+2's first
//      operands and of tile i+1's lse2/delta placed between them.
// Every instruction group is fenced with sched_barrier, so the compiler keeps
// this order.
// ---------------------------------------------------------------------------
constexpr int DK_STAGES = 5;
constexpr int DK_LOADS = 5;  // direct-load instructions per wavefront per query tile
#ifndef DK_AQD
#define DK_AQD 2  // LDS reads of S / dP operands this many MFMA groups ahead
#endif
#ifndef DK_TRD
#define DK_TRD 2  // LDS reads of dV / dK operands this many MFMA groups ahead
#endif

__global__ void __launch_bounds__(256, 1)
fa128_dkdv_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                  const bf16_t* __restrict__ v, int64_t ldv, const float* __restrict__ lse2,
                  const float* __restrict__ delta, const bf16_t* __restrict__ dout,
                  const int64_t* __restrict__ bounds, const int32_t* __restrict__ tiles,
                  int n_tiles, bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int64_t lddv,
                  float* __restrict__ partial, int64_t N, int nq, int nkv, int B, float scale,
                  int* __restrict__ counter, bf16_t* __restrict__ ds,
                  const int64_t* __restrict__ ds_base, int ds_blocks) {
  constexpr int S = DK_STAGES;
  // With `ds`, every 32x32 (query tile, key tile) block of dS^T that the mask
  // allows is stored for the dQ pass (ds_index): buffer stores, so that a
  // block the mask rules out is dropped by the range check (offset past the
  // buffer) rather than branched around.  The buffer is below 2 GiB.
  const __amdgpu_buffer_rsrc_t ds_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      ds, 0, ds ? nq * ds_blocks * DS_BLOCK_BYTES : 0, DS_RSRC_WORD3);
  const uint32_t ds_lane = (uint32_t)((threadIdx.x & 31) * 64 + ((threadIdx.x >> 5) & 1) * 8);
  static_assert(S >= 4, "the ring holds tiles i-1 .. i+2 and the one being loaded");
  __shared__ __attribute__((aligned(1024))) char lds[S][2][QT * ROWB];  // [stage][Q | dO]
  __shared__ __attribute__((aligned(16))) float lds_ld[S][4][2 * QT];   // [stage][wave][lse2 | delta]
  __shared__ int s_item;
  const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Work items: (kv head, key tile), each walking the group's query heads,
  // or, with `partial`, (query head, key tile) writing float32 partials that
  // fa128_dkdv_reduce_kernel sums over the group.  Items differ by more than
  // 30x in work (the first key tiles of a segment see most of its queries)
  // and the hardware hands workgroups to CUs round-robin, so the grid is one
  // workgroup per CU taking items from a counter, heaviest first.  An item's
  // results do not depend on which workgroup takes it.
  const int group = nq / nkv;
  const int heads = partial ? nq : nkv;
  const int n_work = heads * n_tiles;
  for (;;) {
  if (threadIdx.x == 0) s_item = atomicAdd(counter, 1);
  __syncthreads();
  const int item = __builtin_amdgcn_readfirstlane(s_item);
  __syncthreads();  // every lane has read s_item before the next item overwrites it
  if (item >= n_work) break;
  const int bx = item % heads, by = item / heads;
  const int hk = partial ? bx / group : bx;
  const int h_first = partial ? bx : hk * group;
  const int h_end = partial ? h_first + 1 : (hk + 1) * group;
  const int t = n_tiles - 1 - by;
  const int seg = tiles[2 * t], start = tiles[2 * t + 1];
  const int64_t base = bounds[seg];
  const int L = (int)((bounds[seg + 1] - base) / 2);
  const int stream_end = start < L ? L : 2 * L;
  const int k1 = start + 128 < stream_end ? start + 128 : stream_end;
  const int ki = start + wave * 32 + col;
  const bool k_valid = ki < k1;
  const int64_t ldq = (int64_t)nq * HD, ldk = (int64_t)nkv * HD;
  const uint32_t qrow_bytes = (uint32_t)(ldq * 2);
  const float c = scale * FA_LOG2E;

  f32x16_t dkacc[HD / 32], dvacc[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i) {
    mfma_acc_zero(dkacc[i]);
    mfma_acc_zero(dvacc[i]);
  }

  // dS blocks (32-bit: the buffer is below 2 GiB): this wavefront's 32-key
  // tile in its stream, or one no query tile matches when it holds no key,
  // and the first block of the item's first head in this segment
  const int kn = start >= L;
  const int kt = start + 32 * wave < k1 ? ((start - (kn ? L : 0)) >> 5) + wave : (1 << 24);
  const uint32_t ds_item = ds ? (uint32_t)(h_first * ds_blocks + ds_base[seg]) : 0u;
  const int half_blocks = ds_half_blocks(L);

  const Interval2 mine = queries_of_key(ki, k_valid, L, B);
  const Interval2 R = query_ranges(start, k1, L, B);
  // queries allowed for every key of the tile
  const Interval2 first = queries_of_key(start, true, L, B), last = queries_of_key(k1 - 1, true, L, B);
  const bool whole = k1 - start == 128;

  // Cursor (query head h, range r, first row q0) over the query tiles that see
  // this key tile; `more` turns false past the last one.
  // Cursor (query head h, range r, first row q0) over the query tiles that see
  // this key tile, head by head, range 0 then range 1; `more` turns false
  // past the last one.  Branch-free: an exhausted range moves to range 1 of
  // the same head, or to the first range of the next head.
  const bool has1 = R.lo1 < R.hi1;
  const int r_first = R.lo0 < R.hi0 ? 0 : 1, q_first = r_first ? R.lo1 : R.lo0;
  int h = h_first, r = r_first, q0 = q_first;
  bool more = r_first == 0 || has1;
  if (more) {
    // (th, tr, tq): the tile last taken from the cursor.  Past the end it is
    // loaded again, into a stage that is never read, so that every iteration
    // issues DK_LOADS loads and the vmcnt waits stay fixed.
    int th = h, tr = r, tq = q0;
    // Tile descriptors of tiles i .. i+S-1: bit 0 a real tile, bit 1 every key
    // of the key tile sees every row, bit 2 the range, bits 3.. the query
    // head's offset from h_first; and the first row.
    int fl[S], fr[S];
    auto take = [&](int& f, int& row) {
      f = 0;
      if (more) {
        th = h; tr = r; tq = q0;
        const bool full = whole && q0 >= (r ? last.lo1 : last.lo0) &&
                          q0 + QT <= (r ? first.hi1 : first.hi0);
        f = 1 | (full ? 2 : 0) | (r << 2) | ((h - h_first) << 3);
        q0 += QT;
        if (q0 >= (r ? R.hi1 : R.hi0)) {
          const bool to1 = r == 0 && has1;
          h = to1 ? h : h + 1;
          q0 = to1 ? R.lo1 : q_first;
          r = to1 ? 1 : r_first;
          more = h < h_end;
        }
      }
      row = tq;
    };
    // One tile's direct loads: this wavefront's 8 rows of Q and of dO (rows
    // past the range re-read its last row; their products are masked) and its
    // own copy of the tile's 32 lse2 and 32 delta values.  Global addresses are
    // a wave-uniform base plus a 32-bit lane offset; M0 (the LDS destination)
    // is saved once around the five loads.
    const uint32_t lds0 = lds_addr(lds);
    const uint32_t lse_dist = (uint32_t)((const char*)lse2 - (const char*)delta);
    const int rows0 = wave * 8 + (lane >> 4), rows1 = rows0 + 4;
    const uint32_t chunk0 = (uint32_t)((lane & 15) ^ swz(rows0)) << 4;
    const uint32_t chunk1 = (uint32_t)((lane & 15) ^ swz(rows1)) << 4;
    auto issue = [&](int st) {
      const int rel_max = (tr ? R.hi1 : R.hi0) - 1 - tq;
      const int64_t row0 = base + tq;
      const bf16_t* qb = q + row0 * ldq + th * HD;
      const bf16_t* db = dout + row0 * ldq + th * HD;
      const float* lb = delta + (int64_t)th * N + row0;
      const uint32_t off0 = (uint32_t)(rows0 < rel_max ? rows0 : rel_max) * qrow_bytes + chunk0;
      const uint32_t off1 = (uint32_t)(rows1 < rel_max ? rows1 : rel_max) * qrow_bytes + chunk1;
      const uint32_t offl = (uint32_t)(col < rel_max ? col : rel_max) * 4u + (half ? 0u : lse_dist);
      const uint32_t lq = lds0 + (uint32_t)st * (2 * QT * ROWB) + (uint32_t)wave * (8 * ROWB);
      const uint32_t ll = lds_addr(lds_ld) + (uint32_t)(st * 4 + wave) * (2 * QT * 4);
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %[sv], m0\n\t"
          "s_mov_b32 m0, %[lq]\n\t"
          "global_load_lds_dwordx4 %[o0], %[qb]\n\t"
          "s_add_u32 m0, %[lq], %[dq]\n\t"
          "global_load_lds_dwordx4 %[o0], %[db]\n\t"
          "s_add_u32 m0, %[lq], %[r4]\n\t"
          "global_load_lds_dwordx4 %[o1], %[qb]\n\t"
          "s_add_u32 m0, %[lq], %[d4]\n\t"
          "global_load_lds_dwordx4 %[o1], %[db]\n\t"
          "s_mov_b32 m0, %[ll]\n\t"
          "global_load_lds_dword %[ol], %[lb]\n\t"
          "s_mov_b32 m0, %[sv]"
          : [sv] "=&s"(saved)
          : [lq] "s"(lq), [ll] "s"(ll), [o0] "v"(off0), [o1] "v"(off1), [ol] "v"(offl),
            [qb] "s"(qb), [db] "s"(db), [lb] "s"(lb), [dq] "n"(QT * ROWB), [r4] "n"(4 * ROWB),
            [d4] "n"(QT * ROWB + 4 * ROWB)
          : "memory");
    };
    // lse2 and delta of the two elements of S that group kk of the VALU work
    // handles (elements 2kk, 2kk+1 belong to query rows
    // 8 (kk / 2) + 4 half + 2 (kk % 2) + {0, 1} of the tile).
    auto read_pair = [&](int st, int kk, float2& ls, float2& dl) {
      const float* p = lds_ld[st][wave] + 8 * (kk >> 1) + 4 * half + 2 * (kk & 1);
      ls = *reinterpret_cast<const float2*>(p);
      dl = *reinterpret_cast<const float2*>(p + QT);
    };

    // Prologue: tiles 0 .. S-2 into stages 0 .. S-2; K and V fragments.
    bf16x8_t kf[HD / 16], vf[HD / 16];
    take(fl[0], fr[0]);
    issue(0);
    {
      const int64_t kr = base + (k_valid ? ki : k1 - 1);
#pragma unroll
      for (int kk = 0; kk < HD / 16; ++kk) {
        kf[kk] = load_frag(k + kr * ldk + hk * HD + kk * 16 + half * 8);
        vf[kk] = load_frag(v + kr * ldv + hk * HD + kk * 16 + half * 8);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // K, V and this wavefront's share of tile 0
#pragma unroll
    for (int s = 1; s < S - 1; ++s) {
      take(fl[s], fr[s]);
      issue(s);
    }
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(DK_LOADS * (S - 3)) : "memory");
    f32x16_t sacc, pacc;
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      const bf16x8_t a = row_frag(lds[0][0], col, kk * 2 + half);
      const bf16x8_t b = row_frag(lds[0][1], col, kk * 2 + half);
      if (kk == 0) {
        mfma_v0(sacc, a, kf[kk]);
        mfma_v0(pacc, b, vf[kk]);
      } else {
        mfma_v(sacc, a, kf[kk]);
        mfma_v(pacc, b, vf[kk]);
      }
    }
    bf16x8_t aq[HD / 16], ad[HD / 16];  // S / dP A operands of the next tile
#pragma unroll
    for (int kk = 0; kk < DK_AQD; ++kk) {
      aq[kk] = row_frag(lds[1][0], col, 2 * kk + half);
      ad[kk] = row_frag(lds[1][1], col, 2 * kk + half);
    }
    float2 lsa, dla;
    read_pair(0, 0, lsa, dla);
    mfma_acc_settle();  // the first VALU group reads sacc / pacc
    __builtin_amdgcn_sched_barrier(0);

    int cs = 0;  // stage of tile i
    // One iteration: S / dP of tile i in (sacc, pacc) and the lse2 / delta of
    // its first VALU group in (ls0, dl0); leaves tile i+1's in (sn, pn) and
    // (ls1, dl1).  Returns false after the last tile.  The loop alternates
    // the two register sets.
    auto step = [&](f32x16_t& sacc, f32x16_t& pacc, f32x16_t& sn, f32x16_t& pn, float2& ls0,
                    float2& dl0, float2& ls1, float2& dl1) -> bool {
      const int ns = cs + 1 == S ? 0 : cs + 1;
      const int ns2 = ns + 1 == S ? 0 : ns + 1;
      const int ls_stage = cs == 0 ? S - 1 : cs - 1;  // stage of tile i-1 = i+S-1
      const char* qc = lds[cs][0];
      const char* dc = lds[cs][1];
      uint32_t pw[8], sw[8];
      bf16x8_t tv[8], tk[8];  // dO^T / Q^T fragments of dV / dK, index st * 4 + db

      // A: S, dP of tile i+1; P, dS of tile i.
      auto block_a = [&](auto masked_tag) {
        constexpr bool masked = decltype(masked_tag)::value;
        int q_off = 0;
        unsigned q_width = 0;
        if constexpr (masked) {
          const int rr = (fl[0] >> 2) & 1;
          const int qlo = rr ? mine.lo1 : mine.lo0, qhi = rr ? mine.hi1 : mine.hi0;
          q_off = fr[0] + half * 4 - qlo;
          q_width = (unsigned)(qhi - qlo);
        }
        const char* qn = lds[ns][0];
        const char* dn = lds[ns][1];
        float2 lsg = ls0, dlg = dl0;
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk) {
          float2 lsn, dln;
          if (kk + 1 < HD / 16) read_pair(cs, kk + 1, lsn, dln);
          if (kk + DK_AQD < HD / 16) aq[kk + DK_AQD] = row_frag(qn, col, (kk + DK_AQD) * 2 + half);
          if (kk == 0) mfma_v0(sn, aq[kk], kf[kk]);
          else mfma_v(sn, aq[kk], kf[kk]);
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int e = 2 * kk + u;
            float p = fast_exp2(fmaf(sacc[e], c, -(u ? lsg.y : lsg.x)));
            if constexpr (masked)
              if ((unsigned)(q_off + (e >> 2) * 8 + (e & 3)) >= q_width) p = 0.f;
            sacc[e] = p;
            pacc[e] = p * (pacc[e] - (u ? dlg.y : dlg.x));
            if (u == 0 && kk + DK_AQD < HD / 16)
              ad[kk + DK_AQD] = row_frag(dn, col, (kk + DK_AQD) * 2 + half);
            if (u == 0 && kk == 0) mfma_v0(pn, ad[kk], vf[kk]);
            else if (u == 0) mfma_v(pn, ad[kk], vf[kk]);
          }
          pw[kk] = pack2(sacc[2 * kk], sacc[2 * kk + 1]);
          sw[kk] = pack2(pacc[2 * kk], pacc[2 * kk + 1]);
          if (kk == HD / 16 - 1) {
#pragma unroll
            for (int m = 0; m < DK_TRD; ++m) {
              tv[m] = tr_frag(dc, (m >> 2) * 16, (m & 3) * 32, lane);
              tk[m] = tr_frag(qc, (m >> 2) * 16, (m & 3) * 32, lane);
            }
          }
          lsg = lsn;
          dlg = dln;
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if (fl[0] & 2) block_a(std::false_type{});
      else block_a(std::true_type{});
      // The packed P and dS operands of block B are fixed in their registers
      // here, before the barrier: a VALU write of an MFMA source needs wait
      // states that the compiler does not insert ahead of inline-asm MFMAs, so
      // no packing or copy may be left for block B to do.
      bf16x8_t pb[2] = {__builtin_bit_cast(bf16x8_t, make_uint4(pw[0], pw[1], pw[2], pw[3])),
                        __builtin_bit_cast(bf16x8_t, make_uint4(pw[4], pw[5], pw[6], pw[7]))};
      bf16x8_t sb[2] = {__builtin_bit_cast(bf16x8_t, make_uint4(sw[0], sw[1], sw[2], sw[3])),
                        __builtin_bit_cast(bf16x8_t, make_uint4(sw[4], sw[5], sw[6], sw[7]))};
      asm volatile("" : "+v"(pb[0]), "+v"(pb[1]), "+v"(sb[0]), "+v"(sb[1]));

      // Tile i+2 has landed (this wavefront's loads, then every wavefront's);
      // the stage of tile i-1 takes tile i+S-1.
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(DK_LOADS * (S - 4))
                   : "memory");
      __builtin_amdgcn_sched_barrier(0);
      // tile i's dS^T block for this wavefront's keys (rows of 4 consecutive
      // queries 8 j + 4 half + 0..3: dS pairs 2 j, 2 j + 1, half j % 2 of
      // sb[j / 2]), or - when the mask rules the block out - one past the
      // buffer, which drops the stores.  Issued before the next tile's loads,
      // so that the vmcnt wait of the next iteration (which allows those
      // loads to stay in flight) covers these stores as well.
      if (ds) {
        // (branch-free: this loop is issue-bound) the query tile's stream is
        // noisy for a noisy key tile or range 1; ds_allowed / ds_index
        const int qn = kn | ((fl[0] >> 2) & 1);
        const int qt = (fr[0] - (qn ? L : 0)) >> 5;
        const int ok = kn ? (int)(qt == kt) : (int)(kt <= qt - qn);
        const uint32_t blk = ds_item + (uint32_t)((fl[0] >> 3) * ds_blocks) +
                             (uint32_t)(qn ? half_blocks : 0) + (uint32_t)((qt * (qt + 1)) >> 1) +
                             (uint32_t)(kn ? qt : kt);
        const uint32_t ds_off = ok ? blk * DS_BLOCK_BYTES + ds_lane : 0x80000000u;
        typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
        typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x4_t w4 = __builtin_bit_cast(u32x4_t, sb[j >> 1]);
          const u32x2_t w = (j & 1) ? u32x2_t{w4.z, w4.w} : u32x2_t{w4.x, w4.y};
          // non-temporal: dS is read once, by the dQ pass; keeping it out of
          // the caches' normal retention leaves them to the Q / dO tiles
          __builtin_amdgcn_raw_buffer_store_b64(w, ds_rsrc, ds_off + 16u * j, 0, DS_NT);
        }
      }
      take(fl[S - 1], fr[S - 1]);
      issue(ls_stage);
      __builtin_amdgcn_sched_barrier(0);

      // B: dV, dK of tile i; first operands of tile i+2, first lse2 / delta
      // of tile i+1.
      const char* q2 = lds[ns2][0];
      const char* d2 = lds[ns2][1];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        if (m + DK_TRD < 8) {
          tv[m + DK_TRD] = tr_frag(dc, ((m + DK_TRD) >> 2) * 16, ((m + DK_TRD) & 3) * 32, lane);
          tk[m + DK_TRD] = tr_frag(qc, ((m + DK_TRD) >> 2) * 16, ((m + DK_TRD) & 3) * 32, lane);
        }
        mfma_acc(dvacc[m & 3], tv[m], pb[m >> 2]);
        mfma_acc(dkacc[m & 3], tk[m], sb[m >> 2]);
        if (m == 5) read_pair(ns, 0, ls1, dl1);
        // first operands of tile i+2, one k step per group from group 8 - DK_AQD
        if (m >= 8 - DK_AQD) {
          aq[m - (8 - DK_AQD)] = row_frag(q2, col, 2 * (m - (8 - DK_AQD)) + half);
          ad[m - (8 - DK_AQD)] = row_frag(d2, col, 2 * (m - (8 - DK_AQD)) + half);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (!(fl[1] & 1)) return false;
#pragma unroll
      for (int s = 0; s < S - 1; ++s) {
        fl[s] = fl[s + 1];
        fr[s] = fr[s + 1];
      }
      cs = ns;
      return true;
    };
    f32x16_t sn, pn;
    float2 lsb, dlb;
    while (step(sacc, pacc, sn, pn, lsa, dla, lsb, dlb) && step(sn, pn, sacc, pacc, lsb, dlb, lsa, dla)) {
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  mfma_acc_settle();  // the stores below read the accumulators
  if (k_valid && partial) {
    // [2][group][N][nkv * HD]: dK partials, then dV partials
    const int64_t plane = (int64_t)group * N * nkv * HD;
    float* prow = partial + ((int64_t)(h_first % group) * N + base + ki) * (nkv * HD) + hk * HD;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + j * 8 + half * 4;
        *reinterpret_cast<float4*>(prow + d) =
            make_float4(dkacc[db][j * 4] * scale, dkacc[db][j * 4 + 1] * scale,
                        dkacc[db][j * 4 + 2] * scale, dkacc[db][j * 4 + 3] * scale);
        *reinterpret_cast<float4*>(prow + plane + d) =
            make_float4(dvacc[db][j * 4], dvacc[db][j * 4 + 1], dvacc[db][j * 4 + 2],
                        dvacc[db][j * 4 + 3]);
      }
  } else if (k_valid) {
    bf16_t* krow = dk + (base + ki) * ldk + hk * HD;
    bf16_t* vrow = dv + (base + ki) * lddv + hk * HD;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + j * 8 + half * 4;
        *reinterpret_cast<uint2*>(krow + d) =
            make_uint2(pack2(dkacc[db][j * 4] * scale, dkacc[db][j * 4 + 1] * scale),
                       pack2(dkacc[db][j * 4 + 2] * scale, dkacc[db][j * 4 + 3] * scale));
        *reinterpret_cast<uint2*>(vrow + d) =
            make_uint2(pack2(dvacc[db][j * 4], dvacc[db][j * 4 + 1]),
                       pack2(dvacc[db][j * 4 + 2], dvacc[db][j * 4 + 3]));
      }
  }
  }
}

// dK / dV of every key from the group's float32 partials, summed in head
// order (deterministic).  8 consecutive head_dim values per thread; grid x:
// column blocks of a row, y: rows r0 + y, z: dK / dV (no 64-bit division).
__global__ void __launch_bounds__(256)
fa128_dkdv_reduce_kernel(const float* __restrict__ partial, int group, int64_t N, int nkv,
                         bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int64_t lddv,
                         int64_t r0) {
  const int64_t width = (int64_t)nkv * HD;
  const int64_t c = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (c >= width) return;
  const int which = blockIdx.z;  // 0: dK, 1: dV
  const int64_t row = r0 + blockIdx.y;
  const int64_t e = row * width + c;
  const float* src = partial + (int64_t)which * group * N * width + e;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < group; ++g) {
    const float4 a = *reinterpret_cast<const float4*>(src + (int64_t)g * N * width);
    const float4 b = *reinterpret_cast<const float4*>(src + (int64_t)g * N * width + 4);
    acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
    acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
  }
  bf16_t* dst = which ? dv + row * lddv + c : dk + row * width + c;
  Vec8<bf16_t>::store(dst, acc);
}

// ---------------------------------------------------------------------------
// Stored-dS backward (block size 32): prep, dK/dV (storing dS), then dQ.
// ---------------------------------------------------------------------------

// delta[h, r] = sum_e dO[r, h, e] O[r, h, e] and lse2[h, r] = lse[h, r] log2(e)
// (what the dK/dV pass reads when it runs first), and the dK/dV work counter
// zeroed.  16 lanes per (head, row), 8 head_dim values each; a workgroup
// takes 16 heads of one row (grid x: head groups, grid y: rows r0 + y), so it
// reads contiguous pieces of the rows of dO and O, and the row and head need
// no 64-bit division (which took 150 of the flat grid's 275 instructions).
__global__ void __launch_bounds__(256)
fa128_bwd_prep_kernel(const bf16_t* __restrict__ o, const bf16_t* __restrict__ dout,
                      const float* __restrict__ lse, float* __restrict__ delta, int64_t N, int nq,
                      int* __restrict__ counter, int64_t r0) {
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *counter = 0;
  const int h = (int)blockIdx.x * 16 + (int)(threadIdx.x >> 4);
  if (h >= nq) return;
  const int sub = threadIdx.x & 15;
  const int64_t r = r0 + blockIdx.y;
  const int64_t off = r * nq * HD + (int64_t)h * HD + sub * 8;
  float a[8], b[8];
  Vec8<bf16_t>::load(o + off, a);
  Vec8<bf16_t>::load(dout + off, b);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s = fmaf(a[e], b[e], s);
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1) s += __shfl_xor(s, w, 16);
  if (sub == 0) {
    const int64_t hr = (int64_t)h * N + r;  // [head][row] layout
    delta[hr] = s;
    delta[N * nq + hr] = lse[hr] * FA_LOG2E;
  }
}

// dQ = scale * dS K from the stored dS^T blocks: one workgroup per (query
// head, 128-row query tile), walking the tile's keys 32 at a time through a
// ring of DQ_STAGES LDS stages filled by direct loads (K rows and the four
// query tiles' dS^T blocks, both as [32 keys][128] tiles in the swizzled
// layout), DQ_STAGES - 1 key tiles ahead.  Wavefront w accumulates dQ^T for
// head_dim rows 64 (w / 2) .. +64 and query rows 64 (w % 2) .. +64 of the
// tile (2 x 2 MFMA blocks), skipping every (query tile, key tile) pair the
// mask rules out; a ruled-out block's LDS slots hold a stand-in block (the
// head's first) that is never read.
constexpr int DQ_STAGES = 4;
constexpr int DQ_LOADS = 4;  // direct loads per wavefront per key tile

__global__ void __launch_bounds__(256, 2)
fa128_dq_ds_kernel(const bf16_t* __restrict__ k, const bf16_t* __restrict__ ds,
                   const int64_t* __restrict__ ds_base, int64_t ds_blocks,
                   const int64_t* __restrict__ bounds, const int32_t* __restrict__ tiles,
                   bf16_t* __restrict__ dq, int64_t N, int nq, int nkv, float scale) {
  __shared__ __attribute__((aligned(1024))) char lds[DQ_STAGES][2][32 * ROWB];  // [stage][K | dS^T]
  const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.x, hk = h / (nq / nkv);
  const int seg = tiles[2 * blockIdx.y], start = tiles[2 * blockIdx.y + 1];
  const int64_t base = bounds[seg];
  const int L = (int)((bounds[seg + 1] - base) / 2);
  const int stream_end = start < L ? L : 2 * L;
  const int q1 = start + 128 < stream_end ? start + 128 : stream_end;
  const bool qn = start >= L;
  const int qt0 = (start - (qn ? L : 0)) >> 5;  // first 32-row query tile of the tile
  const int nqt = (q1 - start + 31) >> 5;       // its query tiles (1..4)
  const int half_blocks = ds_half_blocks(L);
  // the head's blocks
  const bf16_t* dsh = ds + (int64_t)h * ds_blocks * (DS_BLOCK_BYTES / 2);
  const int64_t seg_blocks = ds_base[seg];
  const int64_t ldk = (int64_t)nkv * HD, ldq = (int64_t)nq * HD;
  const bf16_t* kh = k + hk * HD;
  const int dhb = (wave >> 1) * 2, qb = (wave & 1) * 2;  // first head_dim / query block

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  // Query tile j of the tile (0..3) and key tile kt of range r (0: clean
  // keys, 1: noisy keys) form an allowed block iff kt <= lim[j] (range 0:
  // kt <= q, or kt < q for a noisy query tile q) or kt == eq[j] (range 1);
  // the block is then tri[j] + kt of the head's blocks (ds_index).  -1 for
  // a query tile past the stream.
  int tri[4], lim[4], eq[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = qt0 + j;
    tri[j] = (int)seg_blocks + (qn ? half_blocks : 0) + q * (q + 1) / 2;
    lim[j] = j < nqt ? q - (qn ? 1 : 0) : -1;
    eq[j] = j < nqt && qn ? q : -1;
  }
  // The largest block this tile reads (last query tile, its last key tile)
  // is checked once against the buffer; a table that does not fit reads
  // nothing (dQ 0) rather than past the buffer.
  {
    const int q = qt0 + nqt - 1;
    const bool fits = seg_blocks >= 0 && tri[0] >= 0 && (int64_t)seg_blocks + (qn ? half_blocks : 0) +
                                                            (int64_t)q * (q + 1) / 2 + q < ds_blocks;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lim[j] = fits ? lim[j] : -1;
      eq[j] = fits ? eq[j] : -1;
    }
  }
  // The key tiles: range 0 (clean keys, from key tile 0), then range 1
  // (noisy keys, from tile kt1 = qt0 of the noisy stream, one per query tile
  // of a noisy tile).  In walk order t, query tile j takes the clean key tiles
  // t <= lim[j] (block tri[j] + t) and the noisy key tile t == e[j] (block
  // tri[j] + eq[j]).
  const Interval2 R = key_ranges(start, q1, L, 32);
  const int n0 = R.hi0 > R.lo0 ? (R.hi0 - R.lo0 + 31) / 32 : 0;
  const int n1 = R.hi1 > R.lo1 ? (R.hi1 - R.lo1 + 31) / 32 : 0;
  const int n = n0 + n1;
  const int kt1 = (R.lo1 - L) >> 5;
  int e[4];
  uint32_t b0[4], b1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    e[j] = eq[j] >= 0 ? n0 + (eq[j] - kt1) : -1;
    b0[j] = (uint32_t)tri[j] * DS_BLOCK_BYTES;
    b1[j] = (uint32_t)(tri[j] + eq[j]) * DS_BLOCK_BYTES;
  }
  // this wavefront's two query tiles (qb is 0 or 2)
  const int lim0 = qb ? lim[2] : lim[0], lim1 = qb ? lim[3] : lim[1];
  const int e0 = qb ? e[2] : e[0], e1 = qb ? e[3] : e[1];
  // Per-lane parts of the direct loads, fixed for the whole walk: load i of
  // this wavefront fills tile rows x = 8 wave + 4 i + lane / 16, 16-byte slot
  // lane % 16, i.e. logical chunk c = slot ^ swz(x) (head_dim 8 c.. of the K
  // row; queries 8 c.. of the tile, in query tile c / 4, in the dS^T block).
  uint32_t k_lane[2], ds_lane[2];
  int ds_q[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int x = wave * 8 + 4 * i + (lane >> 4);
    const int c = (lane & 15) ^ swz(x);
    k_lane[i] = (uint32_t)((x * ldk + c * 8) * 2);
    ds_lane[i] = (uint32_t)((x * 32 + (c & 3) * 8) * 2);
    ds_q[i] = c >> 2;
  }
  const uint32_t lds_w = lds_addr(lds) + (uint32_t)(wave * 8 * ROWB);  // this wave's rows
  // Key tile t into stage t % DQ_STAGES: the K rows, and for each query tile
  // of the tile its dS^T block with this key tile (byte offset from the
  // head's first block, a scalar per query tile), or the head's first block
  // when the query tile does not take the key tile.  The four direct loads
  // share one M0 save: M0 is the LDS destination, the wave-uniform base a
  // scalar pair.  Tiles are issued in walk order, so the first K row and the
  // clean-tile block offsets advance by one tile per call.
  int64_t krow = base;       // first K row of the next tile to issue
  uint32_t tb = 0;           // its clean-tile block offset t * 2 KB
  auto issue = [&](int t) {
    if (t == n0) krow = base + L + 32 * kt1;
    uint32_t boff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      boff[j] = t <= lim[j] ? b0[j] + tb : (t == e[j] ? b1[j] : 0u);
    uint32_t off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t b01 = ds_q[i] & 1 ? boff[1] : boff[0];
      const uint32_t b23 = ds_q[i] & 1 ? boff[3] : boff[2];
      off[i] = (ds_q[i] & 2 ? b23 : b01) + ds_lane[i];
    }
    const uint32_t l0 = lds_w + (uint32_t)((t % DQ_STAGES) * (2 * 32 * ROWB));
    if (krow + 32 <= N) {
      const bf16_t* kb = kh + krow * ldk;
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %[sv], m0\n\t"
          "s_mov_b32 m0, %[l0]\n\t"
          "global_load_lds_dwordx4 %[k0], %[kb]\n\t"
          "s_add_u32 m0, %[l0], %[r4]\n\t"
          "global_load_lds_dwordx4 %[k1], %[kb]\n\t"
          "s_add_u32 m0, %[l0], %[dt]\n\t"
          "global_load_lds_dwordx4 %[s0], %[db] nt\n\t"
          "s_add_u32 m0, %[l0], %[dt4]\n\t"
          "global_load_lds_dwordx4 %[s1], %[db] nt\n\t"
          "s_mov_b32 m0, %[sv]"
          : [sv] "=&s"(saved)
          : [l0] "s"(l0), [k0] "v"(k_lane[0]), [k1] "v"(k_lane[1]), [s0] "v"(off[0]),
            [s1] "v"(off[1]), [kb] "s"(kb), [db] "s"(dsh), [r4] "n"(4 * ROWB),
            [dt] "n"(32 * ROWB), [dt4] "n"(36 * ROWB)
          : "memory");
    } else {  // rows past the pack's last row re-read it (their dS is 0)
      const int stg = t % DQ_STAGES;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r0 = wave * 8 + i * 4;
        dload4(lds[stg][0], r0, kh, ldk, krow, N - 1, lane);
        dma16_s_nt(dsh, off[i], lds_addr(lds[stg][1] + r0 * ROWB));
      }
    }
    krow += 32;
    tb += DS_BLOCK_BYTES;
  };
#pragma unroll
  for (int t = 0; t < DQ_STAGES - 1; ++t)
    if (t < n) issue(t);
  for (int t = 0; t < n; ++t) {
    // key tile t has landed (this wavefront's loads, then every
    // wavefront's); later tiles' loads may stay in flight
    const int later = (n - 1 - t) < (DQ_STAGES - 2) ? (n - 1 - t) : (DQ_STAGES - 2);
    if (later >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DQ_LOADS) : "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DQ_LOADS) : "memory");
    else wait_vmem();
    __syncthreads();
    // the stage of key tile t - 1 is free: key tile t + DQ_STAGES - 1 goes there
    if (t + DQ_STAGES - 1 < n) issue(t + DQ_STAGES - 1);
    const char* kt_lds = lds[t % DQ_STAGES][0];
    const char* st_lds = lds[t % DQ_STAGES][1];
    const bool ok0 = t <= lim0 || t == e0, ok1 = t <= lim1 || t == e1;
    if (!ok0 && !ok1) continue;
    // Every operand fragment of the key tile is read before the first MFMA
    // (a ruled-out block's slot holds a stand-in block, harmless to read),
    // so the LDS latency is paid once per tile rather than once per MFMA
    // pair; the memory clobber keeps the reads from sinking into the
    // branches below.
    bf16x8_t fa[2][2], fb[2][2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int rk = st * 16;
      fa[st][0] = tr_frag(kt_lds, rk, dhb * 32, lane);
      fa[st][1] = tr_frag(kt_lds, rk, dhb * 32 + 32, lane);
      fb[st][0] = tr_frag(st_lds, rk, qb * 32, lane);
      fb[st][1] = tr_frag(st_lds, rk, qb * 32 + 32, lane);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      if (ok0) {
        acc[0][0] = mfma(fa[st][0], fb[st][0], acc[0][0]);
        acc[1][0] = mfma(fa[st][1], fb[st][0], acc[1][0]);
      }
      if (ok1) {
        acc[0][1] = mfma(fa[st][0], fb[st][1], acc[0][1]);
        acc[1][1] = mfma(fa[st][1], fb[st][1], acc[1][1]);
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int qi = start + (qb + j) * 32 + col;
    if (qi >= q1) continue;
    bf16_t* row = dq + (base + qi) * ldq + (int64_t)h * HD;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int d = (dhb + i) * 32 + jj * 8 + half * 4;
        *reinterpret_cast<uint2*>(row + d) =
            make_uint2(pack2(acc[i][j][jj * 4] * scale, acc[i][j][jj * 4 + 1] * scale),
                       pack2(acc[i][j][jj * 4 + 2] * scale, acc[i][j][jj * 4 + 3] * scale));
      }
  }
}

// ---------------------------------------------------------------------------
// Launchers (head_dim 128)
// ---------------------------------------------------------------------------

// The dK/dV pass splits its work by query head when (kv head, key tile)
// workgroups would not fill the chip four times over: a single long sequence
// has few key tiles and the first ones see most of the queries.
static bool dkdv_head_split(int64_t n_tiles, int nq, int nkv) {
  return nq > nkv && (int64_t)nkv * n_tiles < 1024;
}

// delta [nq][N], lse * log2(e) [nq][N], the dK/dV work counter (one int in a
// 64-float slot), then (head split) the float32 dK/dV partials
// [2][group][N][nkv*128], then (stored dS) nq * ds_blocks dS^T blocks,
// 256-byte aligned.
constexpr int64_t COUNTER_SLOT = 64;
static int64_t fa128_ds_offset(int64_t N, int nq, int nkv, int64_t n_tiles) {
  const int64_t head = 2 * N * nq + COUNTER_SLOT;
  const int64_t end = dkdv_head_split(n_tiles, nq, nkv) ? head + 2 * N * (int64_t)nq * HD : head;
  return (end + 63) / 64 * 64;
}
// The stored-dS path needs the block size 32 and a dS buffer below 2 GiB (its
// buffer stores take 32-bit offsets).
static bool fa128_ds_path(int64_t nq, int64_t ds_blocks, int64_t block_size) {
  return block_size == 32 && ds_blocks > 0 && nq * ds_blocks * DS_BLOCK_BYTES < (int64_t(1) << 31);
}
int64_t fa128_bwd_workspace(int64_t N, int nq, int nkv, int64_t n_tiles, int64_t ds_blocks) {
  const int64_t off = fa128_ds_offset(N, nq, nkv, n_tiles);
  if (ds_blocks > 0 && nq * ds_blocks * DS_BLOCK_BYTES < (int64_t(1) << 31))
    return off + (int64_t)nq * ds_blocks * (DS_BLOCK_BYTES / 4);
  const int64_t head = 2 * N * nq + COUNTER_SLOT;
  return dkdv_head_split(n_tiles, nq, nkv) ? head + 2 * N * (int64_t)nq * HD : head;
}

int fa128_fwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                     const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* o,
                     float* lse, int64_t N, int nq, int nkv, int B, float scale, hipStream_t st) {
  fa128_fwd_kernel<<<dim3((unsigned)nq, (unsigned)n_tiles), 256, 0, st>>>(
      q, k, v, ldv, bounds, tiles, o, lse, N, nq, nkv, B, scale);
  ALODLM_CHECK_LAUNCH("attention_fwd_fa128");
  return ALODLM_OK;
}

int fa128_bwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                     const float* lse, const bf16_t* o, float* delta, const bf16_t* dout,
                     const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* dq,
                     bf16_t* dk, bf16_t* dv, int64_t lddv, int64_t N, int nq, int nkv, int B,
                     float scale, const int64_t* ds_base, int64_t ds_blocks, hipStream_t st) {
  int* counter = reinterpret_cast<int*>(delta + 2 * N * nq);
  const bool stored = ds_base != nullptr && fa128_ds_path(nq, ds_blocks, B);
  bf16_t* ds = stored ? reinterpret_cast<bf16_t*>(delta + fa128_ds_offset(N, nq, nkv, n_tiles))
                      : nullptr;
  if (stored) {
    // delta, lse * log2(e) and the zeroed work counter for the dK/dV pass,
    // which stores dS for the dQ pass (stream order)
    for (int64_t r0 = 0; r0 < N; r0 += 65535) {  // at most 65535 rows per launch
      const int64_t n = N - r0 < 65535 ? N - r0 : 65535;
      fa128_bwd_prep_kernel<<<dim3(ceil_div_u(nq, 16), (unsigned)n), 256, 0, st>>>(
          o, dout, lse, delta, N, nq, counter, r0);
    }
  } else {
    // the dQ pass writes delta and lse * log2(e), which the dK/dV pass reads
    // (stream order), and zeroes the dK/dV work counter
    fa128_dq_kernel<<<dim3((unsigned)nq, (unsigned)n_tiles), 256, 0, st>>>(
        q, k, v, ldv, lse, o, delta, dout, bounds, tiles, dq, N, nq, nkv, B, scale, counter);
  }
  const float* lse2 = delta + N * nq;
  const bool split = dkdv_head_split(n_tiles, nq, nkv);
  const int64_t items = (split ? nq : nkv) * n_tiles;
  const unsigned grid = (unsigned)(items < device_cus() ? items : device_cus());
  float* partial = split ? delta + 2 * N * nq + COUNTER_SLOT : nullptr;
  fa128_dkdv_kernel<<<grid, 256, 0, st>>>(q, k, v, ldv, lse2, delta, dout, bounds, tiles,
                                          (int)n_tiles, dk, dv, lddv, partial, N, nq, nkv, B,
                                          scale, counter, ds, ds_base, (int)ds_blocks);
  if (split) {
    // a block covers one row's nkv * 16 column groups (at most 256 threads)
    const int64_t per_row = (int64_t)nkv * HD / 8;
    const unsigned threads = (unsigned)(per_row < 256 ? per_row : 256);
    for (int64_t r0 = 0; r0 < N; r0 += 65535) {  // at most 65535 rows per launch
      const int64_t n = N - r0 < 65535 ? N - r0 : 65535;
      fa128_dkdv_reduce_kernel<<<dim3(ceil_div_u(per_row, threads), (unsigned)n, 2), threads, 0,
                                 st>>>(partial, nq / nkv, N, nkv, dk, dv, lddv, r0);
    }
  }
  if (stored)
    fa128_dq_ds_kernel<<<dim3((unsigned)nq, (unsigned)n_tiles), 256, 0, st>>>(
        k, ds, ds_base, ds_blocks, bounds, tiles, dq, N, nq, nkv, scale);
  ALODLM_CHECK_LAUNCH("attention_bwd_fa128");
  return ALODLM_OK;
}
