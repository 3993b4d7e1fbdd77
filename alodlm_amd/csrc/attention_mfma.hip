// bf16 flash attention on gfx950 MFMA under the dual-stream training mask.
//
// Tiles: a 128-row tile never crosses a stream (clean / noisy half) or a
// segment; the host lists them as (segment, in-segment start) pairs.
//
// Forward and dQ: one workgroup = one 128-row query tile of one query head,
// four wavefronts of 32 query rows.  Per 64-key tile the wavefront computes
// S^T = K . Q^T with v_mfma_f32_32x32x16_bf16 (K rows from LDS, Q fragments in
// registers), so that each lane owns one query column: the online softmax is
// lane-local plus one exchange with lane^32, and the probabilities already sit
// in the B-operand layout of O^T += V^T . P^T (keys taken in the permuted order
// 16s + 8(t/4) + 4*half + t%4, matched by the V^T reads).  V^T (and K^T for
// dQ) is staged through LDS transposed by an 8x4 register transpose.
//
// dK/dV: one workgroup = one 128-key tile of one kv head, four wavefronts of
// 32 keys; K and V of the tile stay in LDS, and the workgroup walks the query
// heads of the group and the 64-row query tiles that see the keys, with
// S = Q . K^T so that each lane owns a key.
//
// VALU economy: within one stream pair the mask of a lane is an interval of
// key (or query) indices, so masking is two compares; the softmax runs in the
// log2 domain (one FMA + one v_exp_f32 per score) with a lazily raised
// running maximum (accumulators are rescaled only when the maximum grows by
// more than 2^8); bf16 packing is v_cvt_pk_bf16_f32.  Each kernel prefetches
// the next tile's global loads into registers while it computes the current
// one.
#include "attention_common.h"

// ---------------------------------------------------------------------------
// Register staging of an NR x D tile (rows of stride `ld` in global memory)
// ---------------------------------------------------------------------------
template <int D, int NR>
struct RowStage {  // row-major copy into LDS rows of stride D + 8
  static constexpr int CH = D / 8;
  static constexpr int PER = (NR * CH + FA_THREADS - 1) / FA_THREADS;
  uint4 v[PER];
  __device__ __forceinline__ void load(const bf16_t* g, int64_t ld, int64_t row0, int64_t limit) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int c = threadIdx.x + FA_THREADS * p;
      const int r = c / CH, cc = (c % CH) * 8;
      const bool ok = c < NR * CH && row0 + r < limit;
      const int64_t gr = ok ? row0 + r : row0;
      uint4 x = *reinterpret_cast<const uint4*>(g + gr * ld + cc);
      v[p] = ok ? x : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int c = threadIdx.x + FA_THREADS * p;
      if (c < NR * CH) *reinterpret_cast<uint4*>(lds + (c / CH) * (D + 8) + (c % CH) * 8) = v[p];
    }
  }
};

template <int D, int NR>
struct TStage {  // transposed copy: D rows of stride NR + 8, via 8(row) x 4(col) blocks
  static constexpr int BLK = (NR / 8) * (D / 4);
  static constexpr int PER = (BLK + FA_THREADS - 1) / FA_THREADS;
  uint2 v[PER][8];
  __device__ __forceinline__ void load(const bf16_t* g, int64_t ld, int64_t row0, int64_t limit) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int b = threadIdx.x + FA_THREADS * p;
      const int cq = b % (D / 4), rq = b / (D / 4);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t gr = row0 + rq * 8 + j;
        const bool ok = b < BLK && gr < limit;
        uint2 x = *reinterpret_cast<const uint2*>(g + (ok ? gr : row0) * ld + cq * 4);
        v[p][j] = ok ? x : make_uint2(0, 0);
      }
    }
  }
  __device__ __forceinline__ void store(bf16_t* lds) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int b = threadIdx.x + FA_THREADS * p;
      if (b >= BLK) continue;
      const int cq = b % (D / 4), rq = b / (D / 4);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t a = (c < 2) ? v[p][2 * q].x : v[p][2 * q].y;
          const uint32_t b2 = (c < 2) ? v[p][2 * q + 1].x : v[p][2 * q + 1].y;
          w[q] = (c & 1) ? ((a >> 16) | (b2 & 0xffff0000u)) : ((a & 0xffffu) | (b2 << 16));
        }
        *reinterpret_cast<uint4*>(lds + (cq * 4 + c) * (NR + 8) + rq * 8) =
            make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(FA_THREADS)
fa_fwd_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
              const bf16_t* __restrict__ v, int64_t ldv, const int64_t* __restrict__ bounds,
              const int32_t* __restrict__ tiles, bf16_t* __restrict__ o, float* __restrict__ lse,
              int64_t N, int nq, int nkv, int B, float scale) {
  __shared__ __attribute__((aligned(16))) bf16_t lds_k[FA_KT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_vt[D * (FA_KT + 8)];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, col = lane & 31;
  const int h = blockIdx.y, hk = h / (nq / nkv);
  const int seg = tiles[2 * blockIdx.x], start = tiles[2 * blockIdx.x + 1];
  const int64_t base = bounds[seg];
  const int L = (int)((bounds[seg + 1] - base) / 2);
  const int stream_end = start < L ? L : 2 * L;
  const int q1 = start + 128 < stream_end ? start + 128 : stream_end;
  const int qi = start + wave * 32 + col;
  const bool q_valid = qi < q1;
  const int64_t ldq = (int64_t)nq * D, ldk = (int64_t)nkv * D;
  const float c = scale * FA_LOG2E;

  bf16x8_t qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    if (q_valid) qf[kk] = load_frag(q + (base + qi) * ldq + h * D + kk * 16 + half * 8);
    else qf[kk] = bf16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }
  f32x16_t oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) oacc[i] = zero16();
  float m = -INFINITY, l = 0.f;  // running maximum (log2 units) and sum

  const Interval2 mine = keys_of_query(qi, q_valid, L, B);
  const Interval2 R = key_ranges(start, q1, L, B);
  // keys allowed for every row of the tile (first row: smallest upper bounds,
  // last row: largest lower bound)
  const Interval2 first = keys_of_query(start, true, L, B), last = keys_of_query(q1 - 1, true, L, B);
  int r, k0;
  bool more = range_first(R, r, k0);
  RowStage<D, FA_KT> sk;
  TStage<D, FA_KT> sv;
  if (more) {
    sk.load(k + hk * D, ldk, base + k0, N);
    sv.load(v + hk * D, ldv, base + k0, N);
  }
  while (more) {
    __syncthreads();
    sk.store(lds_k);
    sv.store(lds_vt);
    __syncthreads();
    const int cur_k0 = k0;
    const int klo = r ? mine.lo1 : mine.lo0, khi = r ? mine.hi1 : mine.hi0;
    const bool full = cur_k0 >= (r ? last.lo1 : last.lo0) &&
                      cur_k0 + FA_KT <= (r ? first.hi1 : first.hi0);
    more = range_next(R, FA_KT, r, k0);
    if (more) {
      sk.load(k + hk * D, ldk, base + k0, N);
      sv.load(v + hk * D, ldv, base + k0, N);
    }
    f32x16_t sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sacc[kb] = zero16();
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8_t a = load_frag(lds_k + (kb * 32 + col) * (D + 8) + kk * 16 + half * 8);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sacc[kb], 0, 0, 0);
      }
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
      for (int i = 0; i < D / 32; ++i)
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
    for (int st = 0; st < 4; ++st) {
      const bf16x8_t pb = pack8(sacc[st >> 1], (st & 1) * 8);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const bf16x8_t a = load_split_frag(lds_vt + (db * 32 + col) * (FA_KT + 8) + st * 16 + half * 4);
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, oacc[db], 0, 0, 0);
      }
    }
  }
  if (q_valid) {
    const float inv = 1.0f / l;
    bf16_t* orow = o + (base + qi) * ldq + h * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = db * 32 + j * 8 + half * 4;
        *reinterpret_cast<uint2*>(orow + d) =
            make_uint2(pack2(oacc[db][j * 4] * inv, oacc[db][j * 4 + 1] * inv),
                       pack2(oacc[db][j * 4 + 2] * inv, oacc[db][j * 4 + 3] * inv));
      }
    if (half == 0) lse[(int64_t)h * N + base + qi] = m * FA_LN2 + logf(l);
  }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(FA_THREADS)
fa_dq_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
             const bf16_t* __restrict__ v, int64_t ldv, const float* __restrict__ lse,
             const float* __restrict__ delta, const bf16_t* __restrict__ dout,
             const int64_t* __restrict__ bounds, const int32_t* __restrict__ tiles,
             bf16_t* __restrict__ dq, int64_t N, int nq, int nkv, int B, float scale) {
  __shared__ __attribute__((aligned(16))) bf16_t lds_k[FA_KT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_v[FA_KT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_kt[D * (FA_KT + 8)];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, col = lane & 31;
  const int h = blockIdx.y, hk = h / (nq / nkv);
  const int seg = tiles[2 * blockIdx.x], start = tiles[2 * blockIdx.x + 1];
  const int64_t base = bounds[seg];
  const int L = (int)((bounds[seg + 1] - base) / 2);
  const int stream_end = start < L ? L : 2 * L;
  const int q1 = start + 128 < stream_end ? start + 128 : stream_end;
  const int qi = start + wave * 32 + col;
  const bool q_valid = qi < q1;
  const int64_t ldq = (int64_t)nq * D, ldk = (int64_t)nkv * D;
  const float c = scale * FA_LOG2E;

  bf16x8_t qf[D / 16], df[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    if (q_valid) {
      qf[kk] = load_frag(q + (base + qi) * ldq + h * D + kk * 16 + half * 8);
      df[kk] = load_frag(dout + (base + qi) * ldq + h * D + kk * 16 + half * 8);
    } else {
      qf[kk] = bf16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      df[kk] = qf[kk];
    }
  }
  const float lse2 = q_valid ? lse[(int64_t)h * N + base + qi] * FA_LOG2E : 0.f;
  const float delta_q = q_valid ? delta[(int64_t)h * N + base + qi] : 0.f;
  f32x16_t acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = zero16();

  const Interval2 mine = keys_of_query(qi, q_valid, L, B);
  const Interval2 R = key_ranges(start, q1, L, B);
  const Interval2 first = keys_of_query(start, true, L, B), last = keys_of_query(q1 - 1, true, L, B);
  int r, k0;
  bool more = range_first(R, r, k0);
  RowStage<D, FA_KT> sk, sv;
  TStage<D, FA_KT> skt;
  if (more) {
    sk.load(k + hk * D, ldk, base + k0, N);
    sv.load(v + hk * D, ldv, base + k0, N);
    skt.load(k + hk * D, ldk, base + k0, N);
  }
  while (more) {
    __syncthreads();
    sk.store(lds_k);
    sv.store(lds_v);
    skt.store(lds_kt);
    __syncthreads();
    const int cur_k0 = k0;
    const int klo = r ? mine.lo1 : mine.lo0, khi = r ? mine.hi1 : mine.hi0;
    const bool full = cur_k0 >= (r ? last.lo1 : last.lo0) &&
                      cur_k0 + FA_KT <= (r ? first.hi1 : first.hi0);
    more = range_next(R, FA_KT, r, k0);
    if (more) {
      sk.load(k + hk * D, ldk, base + k0, N);
      sv.load(v + hk * D, ldv, base + k0, N);
      skt.load(k + hk * D, ldk, base + k0, N);
    }
    f32x16_t sacc[2], pacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) { sacc[kb] = zero16(); pacc[kb] = zero16(); }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8_t a = load_frag(lds_k + (kb * 32 + col) * (D + 8) + kk * 16 + half * 8);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sacc[kb], 0, 0, 0);
        const bf16x8_t b = load_frag(lds_v + (kb * 32 + col) * (D + 8) + kk * 16 + half * 8);
        pacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, df[kk], pacc[kb], 0, 0, 0);
      }
    // dS^T = P^T * (dP^T - delta) with P^T = exp(S^T*scale - lse)
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
    for (int st = 0; st < 4; ++st) {
      const bf16x8_t db8 = pack8(sacc[st >> 1], (st & 1) * 8);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const bf16x8_t a = load_split_frag(lds_kt + (db * 32 + col) * (FA_KT + 8) + st * 16 + half * 4);
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, db8, acc[db], 0, 0, 0);
      }
    }
  }
  if (q_valid) {
    bf16_t* row = dq + (base + qi) * ldq + h * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
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
// dK / dV
// ---------------------------------------------------------------------------
template <int D>
__global__ void __launch_bounds__(FA_THREADS)
fa_dkdv_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
               const bf16_t* __restrict__ v, int64_t ldv, const float* __restrict__ lse,
               const float* __restrict__ delta, const bf16_t* __restrict__ dout,
               const int64_t* __restrict__ bounds, const int32_t* __restrict__ tiles,
               bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, int64_t lddv, int64_t N, int nq,
               int nkv, int B, float scale) {
  __shared__ __attribute__((aligned(16))) bf16_t lds_k[128 * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_v[128 * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_q[FA_QT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_do[FA_QT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_qt[D * (FA_QT + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_dot[D * (FA_QT + 8)];
  __shared__ __attribute__((aligned(16))) float lds_lse[FA_QT], lds_delta[FA_QT];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5, col = lane & 31;
  const int hk = blockIdx.y, group = nq / nkv;
  const int seg = tiles[2 * blockIdx.x], start = tiles[2 * blockIdx.x + 1];
  const int64_t base = bounds[seg];
  const int L = (int)((bounds[seg + 1] - base) / 2);
  const int stream_end = start < L ? L : 2 * L;
  const int k1 = start + 128 < stream_end ? start + 128 : stream_end;
  const int ki = start + wave * 32 + col;
  const bool k_valid = ki < k1;
  const int64_t ldq = (int64_t)nq * D, ldk = (int64_t)nkv * D;
  const float c = scale * FA_LOG2E;

  {  // K and V of the key tile, once
    RowStage<D, 128> s;
    s.load(k + hk * D, ldk, base + start, base + k1);
    s.store(lds_k);
    s.load(v + hk * D, ldv, base + start, base + k1);
    s.store(lds_v);
  }
  f32x16_t dkacc[D / 32], dvacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) { dkacc[i] = zero16(); dvacc[i] = zero16(); }

  const Interval2 mine = queries_of_key(ki, k_valid, L, B);
  const Interval2 R = query_ranges(start, k1, L, B);
  // queries allowed for every key of the tile
  const Interval2 first = queries_of_key(start, true, L, B), last = queries_of_key(k1 - 1, true, L, B);
  int r = 0, q0 = 0, h = hk * group;
  bool more = range_first(R, r, q0);
  RowStage<D, FA_QT> sq, sdo;
  TStage<D, FA_QT> sqt, sdot;
  float pre_lse = 0.f, pre_delta = 0.f;
  auto prefetch = [&](int hh, int rr, int qq) {
    const int hi = rr ? R.hi1 : R.hi0;
    const int64_t lim = base + hi;
    sq.load(q + hh * D, ldq, base + qq, lim);
    sdo.load(dout + hh * D, ldq, base + qq, lim);
    sqt.load(q + hh * D, ldq, base + qq, lim);
    sdot.load(dout + hh * D, ldq, base + qq, lim);
    if (threadIdx.x < FA_QT) {
      const bool ok = qq + (int)threadIdx.x < hi;
      const int64_t row = base + qq + (ok ? (int)threadIdx.x : 0);
      const float a = lse[(int64_t)hh * N + row], b = delta[(int64_t)hh * N + row];
      pre_lse = ok ? a * FA_LOG2E : 0.f;
      pre_delta = ok ? b : 0.f;
    }
  };
  if (more) prefetch(h, r, q0);
  while (more) {
    __syncthreads();
    sq.store(lds_q);
    sdo.store(lds_do);
    sqt.store(lds_qt);
    sdot.store(lds_dot);
    if (threadIdx.x < FA_QT) { lds_lse[threadIdx.x] = pre_lse; lds_delta[threadIdx.x] = pre_delta; }
    __syncthreads();
    const int cur_q0 = q0;
    const int qlo = r ? mine.lo1 : mine.lo0, qhi = r ? mine.hi1 : mine.hi0;
    const bool full = k1 - start == 128 && cur_q0 >= (r ? last.lo1 : last.lo0) &&
                      cur_q0 + FA_QT <= (r ? first.hi1 : first.hi0);
    more = range_next(R, FA_QT, r, q0);
    if (!more && h + 1 < (hk + 1) * group) {
      ++h;
      more = range_first(R, r, q0);
    }
    if (more) prefetch(h, r, q0);
    f32x16_t sacc[2], pacc[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) { sacc[qb] = zero16(); pacc[qb] = zero16(); }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const bf16x8_t kb = load_frag(lds_k + (wave * 32 + col) * (D + 8) + kk * 16 + half * 8);
      const bf16x8_t vb = load_frag(lds_v + (wave * 32 + col) * (D + 8) + kk * 16 + half * 8);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const bf16x8_t a = load_frag(lds_q + (qb * 32 + col) * (D + 8) + kk * 16 + half * 8);
        sacc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kb, sacc[qb], 0, 0, 0);
        const bf16x8_t b = load_frag(lds_do + (qb * 32 + col) * (D + 8) + kk * 16 + half * 8);
        pacc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, vb, pacc[qb], 0, 0, 0);
      }
    }
    // S[q, key]: lane owns key column; rows cur_q0 + qb*32 + 8j + 4*half + i
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int qo = qb * 32 + j * 8 + half * 4;
        const float4 ls = *reinterpret_cast<const float4*>(lds_lse + qo);
        const float4 dl = *reinterpret_cast<const float4*>(lds_delta + qo);
        const float lsv[4] = {ls.x, ls.y, ls.z, ls.w}, dlv[4] = {dl.x, dl.y, dl.z, dl.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = j * 4 + i;
          float p = fast_exp2(fmaf(sacc[qb][e], c, -lsv[i]));
          if (!full) {
            const int qq = cur_q0 + qo + i;
            if (qq < qlo || qq >= qhi) p = 0.f;
          }
          sacc[qb][e] = p;
          pacc[qb][e] = p * (pacc[qb][e] - dlv[i]);
        }
      }
#pragma unroll
    for (int st = 0; st < FA_QT / 16; ++st) {
      const bf16x8_t pb = pack8(sacc[st >> 1], (st & 1) * 8);
      const bf16x8_t sb = pack8(pacc[st >> 1], (st & 1) * 8);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const bf16x8_t a = load_split_frag(lds_dot + (db * 32 + col) * (FA_QT + 8) + st * 16 + half * 4);
        dvacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, dvacc[db], 0, 0, 0);
        const bf16x8_t b = load_split_frag(lds_qt + (db * 32 + col) * (FA_QT + 8) + st * 16 + half * 4);
        dkacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, sb, dkacc[db], 0, 0, 0);
      }
    }
  }
  if (k_valid) {
    bf16_t* krow = dk + (base + ki) * ldk + hk * D;
    bf16_t* vrow = dv + (base + ki) * lddv + hk * D;
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
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

// ---------------------------------------------------------------------------
// Launchers (called by the C-ABI entry points in attention.hip)
// ---------------------------------------------------------------------------
int fa_fwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                  const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* o,
                  float* lse, int64_t N, int nq, int nkv, int dh, int B, float scale,
                  hipStream_t st) {
  dim3 grid((unsigned)n_tiles, (unsigned)nq);
  if (dh == 128) fa_fwd_kernel<128><<<grid, FA_THREADS, 0, st>>>(q, k, v, ldv, bounds, tiles, o, lse, N, nq, nkv, B, scale);
  else fa_fwd_kernel<64><<<grid, FA_THREADS, 0, st>>>(q, k, v, ldv, bounds, tiles, o, lse, N, nq, nkv, B, scale);
  ALODLM_CHECK_LAUNCH("attention_fwd_mfma");
  return ALODLM_OK;
}

int fa_bwd_launch(const bf16_t* q, const bf16_t* k, const bf16_t* v, int64_t ldv,
                  const float* lse, const float* delta, const bf16_t* dout,
                  const int64_t* bounds, const int32_t* tiles, int64_t n_tiles, bf16_t* dq,
                  bf16_t* dk, bf16_t* dv, int64_t lddv, int64_t N, int nq, int nkv, int dh,
                  int B, float scale, hipStream_t st) {
  dim3 gq((unsigned)n_tiles, (unsigned)nq), gk((unsigned)n_tiles, (unsigned)nkv);
  if (dh == 128) {
    fa_dq_kernel<128><<<gq, FA_THREADS, 0, st>>>(q, k, v, ldv, lse, delta, dout, bounds, tiles, dq, N, nq, nkv, B, scale);
    fa_dkdv_kernel<128><<<gk, FA_THREADS, 0, st>>>(q, k, v, ldv, lse, delta, dout, bounds, tiles, dk, dv, lddv, N, nq, nkv, B, scale);
  } else {
    fa_dq_kernel<64><<<gq, FA_THREADS, 0, st>>>(q, k, v, ldv, lse, delta, dout, bounds, tiles, dq, N, nq, nkv, B, scale);
    fa_dkdv_kernel<64><<<gk, FA_THREADS, 0, st>>>(q, k, v, ldv, lse, delta, dout, bounds, tiles, dk, dv, lddv, N, nq, nkv, B, scale);
  }
  ALODLM_CHECK_LAUNCH("attention_bwd_mfma");
  return ALODLM_OK;
}
