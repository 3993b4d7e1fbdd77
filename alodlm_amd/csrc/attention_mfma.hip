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
// 32 keys; it loops over the query heads of the group and the 32-row query
// tiles that see the keys, with S = Q . K^T so that each lane owns a key.
//
// Only key tiles that intersect the allowed region are visited; a tile whose
// four corners are allowed skips the per-element mask.
#include "common.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

#define FA_THREADS 256
#define FA_KT 64    // keys per tile (forward / dQ)
#define FA_QT 32    // query rows per tile (dK/dV)

// allowed(q, k) for in-segment dual-stream indices (alodlm/batch.py:23-31)
__device__ __forceinline__ bool dual_allowed(int q, int k, int L, int B) {
  const bool qn = q >= L, kn = k >= L;
  const int qb = (qn ? q - L : q) / B, kb = (kn ? k - L : k) / B;
  return (qb == kb && qn == kn && k <= q) || (kb < qb && !kn);
}

__device__ __forceinline__ bool rect_allowed(int q0, int q1, int k0, int k1, int L, int B) {
  // [q0, q1] x [k0, k1] inclusive, within one stream pair: the corners decide
  return dual_allowed(q0, k0, L, B) && dual_allowed(q0, k1, L, B) &&
         dual_allowed(q1, k0, L, B) && dual_allowed(q1, k1, L, B);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ bf16x8_t load_frag(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

// Two 4-element (8-byte) runs at p and p+8 as one MFMA operand.
__device__ __forceinline__ bf16x8_t load_split_frag(const bf16_t* p) {
  uint2 a = *reinterpret_cast<const uint2*>(p);
  uint2 b = *reinterpret_cast<const uint2*>(p + 8);
  uint4 u = make_uint4(a.x, a.y, b.x, b.y);
  return *reinterpret_cast<bf16x8_t*>(&u);
}

__device__ __forceinline__ bf16x8_t pack8(const float* v) {
  uint4 u;
  u.x = (uint32_t)float_to_bf16(v[0]) | ((uint32_t)float_to_bf16(v[1]) << 16);
  u.y = (uint32_t)float_to_bf16(v[2]) | ((uint32_t)float_to_bf16(v[3]) << 16);
  u.z = (uint32_t)float_to_bf16(v[4]) | ((uint32_t)float_to_bf16(v[5]) << 16);
  u.w = (uint32_t)float_to_bf16(v[6]) | ((uint32_t)float_to_bf16(v[7]) << 16);
  return *reinterpret_cast<bf16x8_t*>(&u);
}

// Stage `nrows` rows of width D (row stride `ld` elements in global memory)
// into LDS rows of stride D + 8.  Rows at or beyond `row_limit` are zero.
template <int D>
__device__ __forceinline__ void stage_rows(bf16_t* lds, const bf16_t* g, int64_t ld, int64_t row0,
                                           int nrows, int64_t row_limit) {
  constexpr int CH = D / 8;
  for (int c = threadIdx.x; c < nrows * CH; c += FA_THREADS) {
    const int r = c / CH, cc = (c % CH) * 8;
    const int64_t gr = row0 + r;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < row_limit) v = *reinterpret_cast<const uint4*>(g + gr * ld + cc);
    *reinterpret_cast<uint4*>(lds + r * (D + 8) + cc) = v;
  }
}

// Stage the transpose of `nrows` x D (rows = keys or queries) into LDS as
// D rows of stride nrows + 8: each thread loads an 8(row) x 4(col) block with
// 8-byte loads and writes four 16-byte runs.
template <int D>
__device__ __forceinline__ void stage_transposed(bf16_t* lds, const bf16_t* g, int64_t ld,
                                                 int64_t row0, int nrows, int64_t row_limit) {
  const int ldt = nrows + 8;
  const int blocks = (nrows / 8) * (D / 4);
  for (int b = threadIdx.x; b < blocks; b += FA_THREADS) {
    const int cq = b % (D / 4), rq = b / (D / 4);
    uint2 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t gr = row0 + rq * 8 + j;
      v[j] = (gr < row_limit) ? *reinterpret_cast<const uint2*>(g + gr * ld + cq * 4)
                              : make_uint2(0, 0);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t w[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t a = (c < 2) ? v[2 * p].x : v[2 * p].y;
        const uint32_t b2 = (c < 2) ? v[2 * p + 1].x : v[2 * p + 1].y;
        w[p] = (c & 1) ? ((a >> 16) | (b2 & 0xffff0000u)) : ((a & 0xffffu) | (b2 << 16));
      }
      *reinterpret_cast<uint4*>(lds + (cq * 4 + c) * ldt + rq * 8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// Key ranges (in-segment) seen by the query tile [q0, q1) of one stream.
__device__ __forceinline__ void fa_key_ranges(int q0, int q1, int L, int B, int* lo, int* hi) {
  if (q0 < L) {
    lo[0] = 0; hi[0] = q1; lo[1] = hi[1] = 0;
  } else {
    const int j0 = q0 - L, j1 = q1 - L;
    const int clean_end = ((j1 - 1) / B) * B;
    lo[0] = 0; hi[0] = clean_end < L ? clean_end : L;
    lo[1] = L + (j0 / B) * B; hi[1] = q1;
  }
}

// Query ranges (in-segment) that see the key tile [k0, k1) of one stream.
__device__ __forceinline__ void fa_query_ranges(int k0, int k1, int L, int B, int* lo, int* hi) {
  if (k0 < L) {
    lo[0] = k0; hi[0] = L;
    const int first = (k0 / B + 1) * B;
    lo[1] = L + (first < L ? first : L); hi[1] = 2 * L;
  } else {
    const int j1 = k1 - L;
    const int end = ((j1 - 1) / B + 1) * B;
    lo[0] = k0; hi[0] = L + (end < L ? end : L);
    lo[1] = hi[1] = 0;
  }
}

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

  bf16x8_t qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    if (q_valid) qf[kk] = load_frag(q + (base + qi) * ldq + h * D + kk * 16 + half * 8);
    else qf[kk] = bf16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }
  f32x16_t oacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) oacc[i] = zero16();
  float m = -INFINITY, l = 0.f;

  int rlo[2], rhi[2];
  fa_key_ranges(start, q1, L, B, rlo, rhi);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    for (int k0 = rlo[r]; k0 < rhi[r]; k0 += FA_KT) {
      __syncthreads();
      stage_rows<D>(lds_k, k + hk * D, ldk, base + k0, FA_KT, N);
      stage_transposed<D>(lds_vt, v + hk * D, ldv, base + k0, FA_KT, N);
      __syncthreads();
      const bool full = k0 + FA_KT <= rhi[r] && rect_allowed(start, q1 - 1, k0, k0 + FA_KT - 1, L, B);
      f32x16_t sacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = zero16();
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const bf16x8_t a = load_frag(lds_k + (kb * 32 + col) * (D + 8) + kk * 16 + half * 8);
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sacc[kb], 0, 0, 0);
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float s = sacc[kb][e] * scale;
          if (!full) {
            const int key = k0 + kb * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
            if (!(q_valid && key < rhi[r] && dual_allowed(qi, key, L, B))) s = -INFINITY;
          }
          sacc[kb][e] = s;
          mx = fmaxf(mx, s);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m, mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float corr = expf(m - m_use);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float p = expf(sacc[kb][e] - m_use);
          sacc[kb][e] = p;
          rs += p;
        }
      rs += __shfl_xor(rs, 32, 64);
      l = l * corr + rs;
      m = m_new;
#pragma unroll
      for (int i = 0; i < D / 32; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[i][e] *= corr;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        float pv[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) pv[t] = sacc[st >> 1][(st & 1) * 8 + t];
        const bf16x8_t pb = pack8(pv);
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          const bf16x8_t a = load_split_frag(lds_vt + (db * 32 + col) * (FA_KT + 8) + st * 16 + half * 4);
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, oacc[db], 0, 0, 0);
        }
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
        uint2 w;
        w.x = (uint32_t)float_to_bf16(oacc[db][j * 4] * inv) |
              ((uint32_t)float_to_bf16(oacc[db][j * 4 + 1] * inv) << 16);
        w.y = (uint32_t)float_to_bf16(oacc[db][j * 4 + 2] * inv) |
              ((uint32_t)float_to_bf16(oacc[db][j * 4 + 3] * inv) << 16);
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
    if (half == 0) lse[(int64_t)h * N + base + qi] = m + logf(l);
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
  const float lse_q = q_valid ? lse[(int64_t)h * N + base + qi] : 0.f;
  const float delta_q = q_valid ? delta[(int64_t)h * N + base + qi] : 0.f;
  f32x16_t acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = zero16();

  int rlo[2], rhi[2];
  fa_key_ranges(start, q1, L, B, rlo, rhi);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    for (int k0 = rlo[r]; k0 < rhi[r]; k0 += FA_KT) {
      __syncthreads();
      stage_rows<D>(lds_k, k + hk * D, ldk, base + k0, FA_KT, N);
      stage_rows<D>(lds_v, v + hk * D, ldv, base + k0, FA_KT, N);
      stage_transposed<D>(lds_kt, k + hk * D, ldk, base + k0, FA_KT, N);
      __syncthreads();
      const bool full = k0 + FA_KT <= rhi[r] && rect_allowed(start, q1 - 1, k0, k0 + FA_KT - 1, L, B);
      f32x16_t sacc[2], pacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[kb] = zero16();
        pacc[kb] = zero16();
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const bf16x8_t a = load_frag(lds_k + (kb * 32 + col) * (D + 8) + kk * 16 + half * 8);
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sacc[kb], 0, 0, 0);
          const bf16x8_t b = load_frag(lds_v + (kb * 32 + col) * (D + 8) + kk * 16 + half * 8);
          pacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, df[kk], pacc[kb], 0, 0, 0);
        }
      }
      // dS^T = P^T * (dP^T - delta) with P^T = exp(S^T*scale - lse)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          bool ok = q_valid;
          if (!full) {
            const int key = k0 + kb * 32 + (e >> 2) * 8 + half * 4 + (e & 3);
            ok = ok && key < rhi[r] && dual_allowed(qi, key, L, B);
          }
          const float p = ok ? expf(sacc[kb][e] * scale - lse_q) : 0.f;
          sacc[kb][e] = p * (pacc[kb][e] - delta_q);
        }
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        float dv[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) dv[t] = sacc[st >> 1][(st & 1) * 8 + t];
        const bf16x8_t db8 = pack8(dv);
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          const bf16x8_t a = load_split_frag(lds_kt + (db * 32 + col) * (FA_KT + 8) + st * 16 + half * 4);
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, db8, acc[db], 0, 0, 0);
        }
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
        uint2 w;
        w.x = (uint32_t)float_to_bf16(acc[db][j * 4] * scale) |
              ((uint32_t)float_to_bf16(acc[db][j * 4 + 1] * scale) << 16);
        w.y = (uint32_t)float_to_bf16(acc[db][j * 4 + 2] * scale) |
              ((uint32_t)float_to_bf16(acc[db][j * 4 + 3] * scale) << 16);
        *reinterpret_cast<uint2*>(row + d) = w;
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
  __shared__ __attribute__((aligned(16))) bf16_t lds_q[FA_QT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_do[FA_QT * (D + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_qt[D * (FA_QT + 8)];
  __shared__ __attribute__((aligned(16))) bf16_t lds_dot[D * (FA_QT + 8)];
  __shared__ float lds_lse[FA_QT], lds_delta[FA_QT];
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

  bf16x8_t kf[D / 16], vf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    if (k_valid) {
      kf[kk] = load_frag(k + (base + ki) * ldk + hk * D + kk * 16 + half * 8);
      vf[kk] = load_frag(v + (base + ki) * ldv + hk * D + kk * 16 + half * 8);
    } else {
      kf[kk] = bf16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      vf[kk] = kf[kk];
    }
  }
  f32x16_t dkacc[D / 32], dvacc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) { dkacc[i] = zero16(); dvacc[i] = zero16(); }

  int rlo[2], rhi[2];
  fa_query_ranges(start, k1, L, B, rlo, rhi);
  for (int h = hk * group; h < (hk + 1) * group; ++h) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      for (int q0 = rlo[r]; q0 < rhi[r]; q0 += FA_QT) {
        __syncthreads();
        stage_rows<D>(lds_q, q + h * D, ldq, base + q0, FA_QT, N);
        stage_rows<D>(lds_do, dout + h * D, ldq, base + q0, FA_QT, N);
        stage_transposed<D>(lds_qt, q + h * D, ldq, base + q0, FA_QT, N);
        stage_transposed<D>(lds_dot, dout + h * D, ldq, base + q0, FA_QT, N);
        if (threadIdx.x < FA_QT) {
          const int64_t row = base + q0 + threadIdx.x;
          const bool ok = q0 + (int)threadIdx.x < rhi[r];
          lds_lse[threadIdx.x] = ok ? lse[(int64_t)h * N + row] : 0.f;
          lds_delta[threadIdx.x] = ok ? delta[(int64_t)h * N + row] : 0.f;
        }
        __syncthreads();
        const bool full = q0 + FA_QT <= rhi[r] && start + 128 <= k1 &&
                          rect_allowed(q0, q0 + FA_QT - 1, start, k1 - 1, L, B);
        f32x16_t sacc = zero16(), pacc = zero16();
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const bf16x8_t a = load_frag(lds_q + col * (D + 8) + kk * 16 + half * 8);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kf[kk], sacc, 0, 0, 0);
          const bf16x8_t b = load_frag(lds_do + col * (D + 8) + kk * 16 + half * 8);
          pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, vf[kk], pacc, 0, 0, 0);
        }
        // S[q, key]: lane owns key column; rows q0 + 8j + 4*half + i
        float pv[16], dsv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int qo = (e >> 2) * 8 + half * 4 + (e & 3);
          bool ok = k_valid;
          if (!full) ok = ok && q0 + qo < rhi[r] && dual_allowed(q0 + qo, ki, L, B);
          const float p = ok ? expf(sacc[e] * scale - lds_lse[qo]) : 0.f;
          pv[e] = p;
          dsv[e] = p * (pacc[e] - lds_delta[qo]);
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const bf16x8_t pb = pack8(pv + st * 8);
          const bf16x8_t sb = pack8(dsv + st * 8);
#pragma unroll
          for (int db = 0; db < D / 32; ++db) {
            const bf16x8_t a = load_split_frag(lds_dot + (db * 32 + col) * (FA_QT + 8) + st * 16 + half * 4);
            dvacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, dvacc[db], 0, 0, 0);
            const bf16x8_t b = load_split_frag(lds_qt + (db * 32 + col) * (FA_QT + 8) + st * 16 + half * 4);
            dkacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, sb, dkacc[db], 0, 0, 0);
          }
        }
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
        uint2 a, b;
        a.x = (uint32_t)float_to_bf16(dkacc[db][j * 4] * scale) |
              ((uint32_t)float_to_bf16(dkacc[db][j * 4 + 1] * scale) << 16);
        a.y = (uint32_t)float_to_bf16(dkacc[db][j * 4 + 2] * scale) |
              ((uint32_t)float_to_bf16(dkacc[db][j * 4 + 3] * scale) << 16);
        b.x = (uint32_t)float_to_bf16(dvacc[db][j * 4]) |
              ((uint32_t)float_to_bf16(dvacc[db][j * 4 + 1]) << 16);
        b.y = (uint32_t)float_to_bf16(dvacc[db][j * 4 + 2]) |
              ((uint32_t)float_to_bf16(dvacc[db][j * 4 + 3]) << 16);
        *reinterpret_cast<uint2*>(krow + d) = a;
        *reinterpret_cast<uint2*>(vrow + d) = b;
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
