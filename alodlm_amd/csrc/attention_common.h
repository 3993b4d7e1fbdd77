// Shared pieces of the MFMA attention kernels: fragment types and packing,
// and the dual-stream mask of alodlm/batch.py:23-31 as key/query intervals.
#pragma once

#include "common.h"

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

#define FA_THREADS 256
#define FA_KT 64    // keys per tile (forward / dQ)
#define FA_QT 64    // query rows per tile (dK/dV)
#define FA_LOG2E 1.4426950408889634f
#define FA_LN2 0.6931471805599453f
#define FA_RESCALE 8.0f  // log2 headroom before the running maximum is raised

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

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return pack_bf16x2(a, b);
}

// Elements [off, off + 8) of an accumulator as one bf16 MFMA operand.
__device__ __forceinline__ bf16x8_t pack8(const f32x16_t& v, int off) {
  uint4 u = make_uint4(pack2(v[off], v[off + 1]), pack2(v[off + 2], v[off + 3]),
                       pack2(v[off + 4], v[off + 5]), pack2(v[off + 6], v[off + 7]));
  return *reinterpret_cast<bf16x8_t*>(&u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }


// ---------------------------------------------------------------------------
// Mask as intervals (alodlm/batch.py:23-31).  For a query row q (in-segment
// index) the allowed keys form one interval per stream:
//   clean q:            clean keys [0, q]
//   noisy q, block b:   clean keys [0, b*B) and noisy keys [L + b*B, q]
// and for a key k the allowed queries form one interval per stream:
//   clean k, block b:   clean queries [k, L) and noisy queries [L + (b+1)*B, 2L)
//   noisy k, block b:   noisy queries [k, L + (b+1)*B)
// (b*B and (b+1)*B clamped to L).  Range 0 is the clean key (query) stream of
// a tile, range 1 the noisy one.
// ---------------------------------------------------------------------------
struct Interval2 { int lo0, hi0, lo1, hi1; };

__device__ __forceinline__ Interval2 keys_of_query(int q, bool valid, int L, int B) {
  Interval2 r = {0, 0, 0, 0};
  if (!valid) return r;
  if (q < L) { r.hi0 = q + 1; return r; }
  const int bb = ((q - L) / B) * B;
  r.hi0 = bb < L ? bb : L;
  r.lo1 = L + bb;
  r.hi1 = q + 1;
  return r;
}

__device__ __forceinline__ Interval2 queries_of_key(int k, bool valid, int L, int B) {
  Interval2 r = {0, 0, 0, 0};
  if (!valid) return r;
  if (k < L) {
    const int nb = (k / B + 1) * B;
    r.lo0 = k; r.hi0 = L;
    r.lo1 = L + (nb < L ? nb : L); r.hi1 = 2 * L;
    return r;
  }
  const int nb = ((k - L) / B + 1) * B;
  r.lo0 = k; r.hi0 = L + (nb < L ? nb : L);
  return r;
}

// Tile ranges: keys seen by the query tile [q0, q1), queries that see the key
// tile [k0, k1) - the union of the lane intervals.
__device__ __forceinline__ Interval2 key_ranges(int q0, int q1, int L, int B) {
  Interval2 a = keys_of_query(q1 - 1, true, L, B);  // the last row sees the most keys
  if (q0 >= L) a.lo1 = keys_of_query(q0, true, L, B).lo1;
  return a;
}
__device__ __forceinline__ Interval2 query_ranges(int k0, int k1, int L, int B) {
  Interval2 a = queries_of_key(k0, true, L, B);  // the first key is seen by the most queries
  if (k0 >= L) a.hi0 = queries_of_key(k1 - 1, true, L, B).hi0;
  return a;
}

// Walk the tiles of the two ranges.
__device__ __forceinline__ bool range_first(const Interval2& R, int& r, int& pos) {
  r = 0;
  pos = R.lo0;
  if (pos < R.hi0) return true;
  r = 1;
  pos = R.lo1;
  return pos < R.hi1;
}
__device__ __forceinline__ bool range_next(const Interval2& R, int step, int& r, int& pos) {
  pos += step;
  if (pos < (r ? R.hi1 : R.hi0)) return true;
  if (r == 1) return false;
  r = 1;
  pos = R.lo1;
  return pos < R.hi1;
}
