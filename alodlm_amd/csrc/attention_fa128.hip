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
  auto issue = [&](int stg, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r0 = wave * 16 + i * 4;
      dload4(lds[stg][0], r0, kh, ldk, base + k0, N - 1, lane);
      dload4(lds[stg][1], r0, vh, ldv, base + k0, N - 1, lane);
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
                int nkv, int B, float scale) {
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
  auto issue = [&](int stg, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r0 = wave * 16 + i * 4;
      dload4(lds[stg][0], r0, kh, ldk, base + k0, N - 1, lane);
      dload4(lds[stg][1], r0, vh, ldv, base + k0, N - 1, lane);
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
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256, 2)
fa128_dkdv_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                  const bf16_t* __restrict__ v, int64_t ldv, const float* __restrict__ lse2,
                  const float* __restrict__ delta, const bf16_t* __restrict__ dout,
                  const int64_t* __restrict__ bounds, const int32_t* __restrict__ tiles,
                  int n_tiles, bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int64_t lddv,
                  float* __restrict__ partial, int64_t N, int nq, int nkv, int B, float scale) {
  __shared__ __attribute__((aligned(1024))) char lds[2][2][QT * ROWB];  // [stage][Q | dO]
  __shared__ __attribute__((aligned(1024))) char lds_v[128 * ROWB];     // V of the key tile
  __shared__ __attribute__((aligned(16))) float lds_ld[2][2 * QT];      // [stage][lse2 | delta]
  const int lane = threadIdx.x & 63, half = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // One workgroup per (kv head, key tile) walking the group's query heads, or,
  // with `partial`, one per (query head, key tile) writing float32 partials
  // that fa128_dkdv_reduce_kernel sums over the group.
  const int group = nq / nkv;
  const int hk = partial ? (int)blockIdx.x / group : (int)blockIdx.x;
  const int h_first = partial ? (int)blockIdx.x : hk * group;
  const int h_end = partial ? h_first + 1 : (hk + 1) * group;
  const int t = n_tiles - 1 - (int)blockIdx.y;
  const int seg = tiles[2 * t], start = tiles[2 * t + 1];
  const int64_t base = bounds[seg];
  const int L = (int)((bounds[seg + 1] - base) / 2);
  const int stream_end = start < L ? L : 2 * L;
  const int k1 = start + 128 < stream_end ? start + 128 : stream_end;
  const int ki = start + wave * 32 + col;
  const bool k_valid = ki < k1;
  const int64_t ldq = (int64_t)nq * HD, ldk = (int64_t)nkv * HD;
  const float c = scale * FA_LOG2E;

  // K of this wavefront's 32 keys as B operands in registers (lane = key, 8 of
  // head_dim per k step); V of the tile's 128 keys in LDS (same operand reads).
  bf16x8_t kf[HD / 16];
  {
    const int64_t kr = base + (k_valid ? ki : k1 - 1);
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) kf[kk] = load_frag(k + kr * ldk + hk * HD + kk * 16 + half * 8);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dload4(lds_v, wave * 32 + i * 4, v + hk * HD, ldv, base + start, base + k1 - 1, lane);
  }
  f32x16_t dkacc[HD / 32], dvacc[HD / 32];
#pragma unroll
  for (int i = 0; i < HD / 32; ++i) { dkacc[i] = zero16(); dvacc[i] = zero16(); }

  const Interval2 mine = queries_of_key(ki, k_valid, L, B);
  const Interval2 R = query_ranges(start, k1, L, B);
  // queries allowed for every key of the tile
  const Interval2 first = queries_of_key(start, true, L, B), last = queries_of_key(k1 - 1, true, L, B);
  auto issue = [&](int stg, int hh, int rr, int qq) {
    const int64_t gmax = base + (rr ? R.hi1 : R.hi0) - 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = wave * 8 + i * 4;
      dload4(lds[stg][0], r0, q + hh * HD, ldq, base + qq, gmax, lane);
      dload4(lds[stg][1], r0, dout + hh * HD, ldq, base + qq, gmax, lane);
    }
    if (wave == 0) {  // lse2 (lanes 0-31) and delta (lanes 32-63) of the tile's rows
      int64_t row = base + qq + col;
      row = row < gmax ? row : gmax;
      const float* src = (half ? delta : lse2) + (int64_t)hh * N + row;
      dma4_v(src, lds_addr(lds_ld[stg]));
    }
  };
  int r = 0, q0 = 0, h = h_first;
  bool more = range_first(R, r, q0);
  __builtin_amdgcn_s_waitcnt(0);
  if (more) issue(0, h, r, q0);
  int stg = 0;
  while (more) {
    wait_vmem();
    __syncthreads();
    const int cur_q0 = q0;
    const int qlo = r ? mine.lo1 : mine.lo0, qhi = r ? mine.hi1 : mine.hi0;
    const bool full = k1 - start == 128 && cur_q0 >= (r ? last.lo1 : last.lo0) &&
                      cur_q0 + QT <= (r ? first.hi1 : first.hi0);
    more = range_next(R, QT, r, q0);
    if (!more && h + 1 < h_end) {
      ++h;
      more = range_first(R, r, q0);
    }
    if (more) issue(stg ^ 1, h, r, q0);
    const char* qt = lds[stg][0];
    const char* dt = lds[stg][1];
    f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
    for (int kk = 0; kk < HD / 16; ++kk) {
      sacc = mfma(row_frag(qt, col, kk * 2 + half), kf[kk], sacc);
      pacc = mfma(row_frag(dt, col, kk * 2 + half), row_frag(lds_v, wave * 32 + col, kk * 2 + half), pacc);
    }
    // S[q, key]: lane owns the key column; element e is query row 8(e/4) + 4*half + e%4.
    // Query qq is allowed iff (unsigned)(qq - qlo) < qhi - qlo; for a tile every
    // key sees whole the bound is set so that the test always passes (one add,
    // compare and select per element, no second copy of the loop body).
    const int q_off = full ? 0 : cur_q0 + half * 4 - qlo;
    const unsigned q_width = full ? 0xffffffffu : (unsigned)(qhi - qlo);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int qo = j * 8 + half * 4;
      const float4 ls = *reinterpret_cast<const float4*>(&lds_ld[stg][qo]);
      const float4 dl = *reinterpret_cast<const float4*>(&lds_ld[stg][QT + qo]);
      const float lsv[4] = {ls.x, ls.y, ls.z, ls.w}, dlv[4] = {dl.x, dl.y, dl.z, dl.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = j * 4 + i;
        float p = fast_exp2(fmaf(sacc[e], c, -lsv[i]));
        if ((unsigned)(q_off + j * 8 + i) >= q_width) p = 0.f;
        sacc[e] = p;
        pacc[e] = p * (pacc[e] - dlv[i]);
      }
    }
#pragma unroll
    for (int st = 0; st < QT / 16; ++st) {
      const bf16x8_t pb = pack8(sacc, st * 8);
      const bf16x8_t sb = pack8(pacc, st * 8);
#pragma unroll
      for (int db = 0; db < HD / 32; ++db) {
        dvacc[db] = mfma(tr_frag(dt, st * 16, db * 32, lane), pb, dvacc[db]);
        dkacc[db] = mfma(tr_frag(qt, st * 16, db * 32, lane), sb, dkacc[db]);
      }
    }
    stg ^= 1;
  }
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

// dK / dV of every key from the group's float32 partials, summed in head
// order (deterministic).  8 consecutive head_dim values per thread.
__global__ void __launch_bounds__(256)
fa128_dkdv_reduce_kernel(const float* __restrict__ partial, int group, int64_t N, int nkv,
                         bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int64_t lddv) {
  const int64_t width = (int64_t)nkv * HD;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= 2 * N * width) return;
  const int which = i >= N * width;  // 0: dK, 1: dV
  const int64_t e = which ? i - N * width : i;
  const int64_t row = e / width, c = e % width;
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
// Launchers (head_dim 128)
// ---------------------------------------------------------------------------

// The dK/dV pass splits its work by query head when (kv head, key tile)
// workgroups would not fill the chip four times over: a single long sequence
// has few key tiles and the first ones see most of the queries.
static bool dkdv_head_split(int64_t n_tiles, int nq, int nkv) {
  return nq > nkv && (int64_t)nkv * n_tiles < 1024;
}

int64_t fa128_bwd_workspace(int64_t N, int nq, int nkv, int64_t n_tiles) {
  // delta [nq][N], lse * log2(e) [nq][N], then (head split) the float32 dK/dV
  // partials [2][group][N][nkv*128]
  const int64_t delta = 2 * N * nq;
  return dkdv_head_split(n_tiles, nq, nkv) ? delta + 2 * N * (int64_t)nq * HD : delta;
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
                     float scale, hipStream_t st) {
  // the dQ pass writes delta and lse * log2(e), which the dK/dV pass reads
  // (stream order)
  fa128_dq_kernel<<<dim3((unsigned)nq, (unsigned)n_tiles), 256, 0, st>>>(
      q, k, v, ldv, lse, o, delta, dout, bounds, tiles, dq, N, nq, nkv, B, scale);
  const float* lse2 = delta + N * nq;
  if (dkdv_head_split(n_tiles, nq, nkv)) {
    float* partial = delta + 2 * N * nq;
    fa128_dkdv_kernel<<<dim3((unsigned)nq, (unsigned)n_tiles), 256, 0, st>>>(
        q, k, v, ldv, lse2, delta, dout, bounds, tiles, (int)n_tiles, dk, dv, lddv, partial, N,
        nq, nkv, B, scale);
    fa128_dkdv_reduce_kernel<<<ceil_div_u(2 * N * nkv * HD / 8, 256), 256, 0, st>>>(
        partial, nq / nkv, N, nkv, dk, dv, lddv);
  } else {
    fa128_dkdv_kernel<<<dim3((unsigned)nkv, (unsigned)n_tiles), 256, 0, st>>>(
        q, k, v, ldv, lse2, delta, dout, bounds, tiles, (int)n_tiles, dk, dv, lddv, nullptr, N,
        nq, nkv, B, scale);
  }
  ALODLM_CHECK_LAUNCH("attention_bwd_fa128");
  return ALODLM_OK;
}
