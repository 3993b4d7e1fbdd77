// q_norm / k_norm fused with the rotary embedding, forward and backward
// (alodlm/model.py:41-46,58; [tf] modeling_qwen3.py:59-64,126-144).
//
// One wavefront owns one row and walks its nq + nkv heads; a lane owns the
// rotary pairs (i, i + dh/2) for i = lane, lane + 64 (dh <= 256), so the
// angle pos * inv_freq[i] and its cos/sin are evaluated once per row and
// reused by every head.  cos/sin are rounded to the storage type like the
// reference's rotary table, and q*cos, rotate(q)*sin and their sum each round
// to the storage type.
#include "common.h"
#include "norm.h"

#include <type_traits>

#define ROPE_WAVES 4
#define ROPE_MAX_T 2  // pairs per lane: dh/2 <= 128

// The rotation of element pair (i, i + dh/2) of a row: cos/sin of the first
// and of the second element.  From positions, both halves share the angle
// pos * inv_freq[i] ([tf] modeling_qwen3.py:126-137 builds cat(freqs, freqs));
// from caller tables ([rows, dh] in the storage type, alodlm/model.py:41-46)
// each element takes its own entry.
template <typename T, bool TAB>
__device__ __forceinline__ void rope_pair(const int64_t* positions, const float* inv_freq,
                                          const T* cos_tab, const T* sin_tab, int64_t row,
                                          int i, int dh, float& ca, float& cb, float& sa,
                                          float& sb) {
  if (TAB) {
    const int64_t base = row * dh;
    ca = Elem<T>::load(cos_tab, base + i); cb = Elem<T>::load(cos_tab, base + i + dh / 2);
    sa = Elem<T>::load(sin_tab, base + i); sb = Elem<T>::load(sin_tab, base + i + dh / 2);
  } else {
    const float ang = (float)positions[row] * inv_freq[i];
    ca = cb = Elem<T>::round(cosf(ang));
    sa = sb = Elem<T>::round(sinf(ang));
  }
}

template <typename T, bool TAB>
__global__ void __launch_bounds__(64 * ROPE_WAVES)
qknorm_rope_fwd_kernel(const T* __restrict__ qkv, const T* __restrict__ wq, const T* __restrict__ wk,
                       const int64_t* __restrict__ positions, const float* __restrict__ inv_freq,
                       const T* __restrict__ cos_tab, const T* __restrict__ sin_tab,
                       T* __restrict__ q_out, T* __restrict__ k_out, int64_t rows, int nq, int nkv,
                       int dh, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROPE_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int half = dh / 2;
  float csa[ROPE_MAX_T], csb[ROPE_MAX_T], sna[ROPE_MAX_T], snb[ROPE_MAX_T];
  float wqa[ROPE_MAX_T], wqb[ROPE_MAX_T], wka[ROPE_MAX_T], wkb[ROPE_MAX_T];
#pragma unroll
  for (int t = 0; t < ROPE_MAX_T; ++t) {
    const int i = lane + 64 * t;
    if (i < half) {
      rope_pair<T, TAB>(positions, inv_freq, cos_tab, sin_tab, row, i, dh, csa[t], csb[t],
                        sna[t], snb[t]);
      wqa[t] = Elem<T>::load(wq, i); wqb[t] = Elem<T>::load(wq, i + half);
      wka[t] = Elem<T>::load(wk, i); wkb[t] = Elem<T>::load(wk, i + half);
    }
  }
  const T* src = qkv + row * (int64_t)(nq + 2 * nkv) * dh;
  for (int head = 0; head < nq + nkv; ++head) {
    const bool is_q = head < nq;
    const T* x = src + head * dh;
    T* dst = is_q ? q_out + (row * nq + head) * dh : k_out + (row * nkv + head - nq) * dh;
    float xa[ROPE_MAX_T], xb[ROPE_MAX_T];
    float ss = 0.f;
#pragma unroll
    for (int t = 0; t < ROPE_MAX_T; ++t) {
      const int i = lane + 64 * t;
      xa[t] = xb[t] = 0.f;
      if (i < half) {
        xa[t] = Elem<T>::load(x, i);
        xb[t] = Elem<T>::load(x, i + half);
        ss += xa[t] * xa[t] + xb[t] * xb[t];
      }
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)dh + eps);
#pragma unroll
    for (int t = 0; t < ROPE_MAX_T; ++t) {
      const int i = lane + 64 * t;
      if (i < half) {
        const float a = Elem<T>::round((is_q ? wqa[t] : wka[t]) * Elem<T>::round(xa[t] * r));
        const float b = Elem<T>::round((is_q ? wqb[t] : wkb[t]) * Elem<T>::round(xb[t] * r));
        Elem<T>::store(dst, i, Elem<T>::round(a * csa[t]) + Elem<T>::round(-b * sna[t]));
        Elem<T>::store(dst, i + half, Elem<T>::round(b * csb[t]) + Elem<T>::round(a * snb[t]));
      }
    }
  }
}

// Backward: dt = rotary^T d(out), then the RMSNorm backward over dh.  Per-lane
// norm-weight partials stay in registers; the block writes one partial row
// [q grads (dh) | k grads (dh)].

template <typename T, bool TAB>
__global__ void __launch_bounds__(64 * ROPE_WAVES)
qknorm_rope_bwd_kernel(const T* __restrict__ dq, const T* __restrict__ dk, const T* __restrict__ qkv,
                       const T* __restrict__ wq, const T* __restrict__ wk,
                       const int64_t* __restrict__ positions, const float* __restrict__ inv_freq,
                       const T* __restrict__ cos_tab, const T* __restrict__ sin_tab,
                       T* __restrict__ dqkv, float* __restrict__ partial, int64_t rows, int nq,
                       int nkv, int dh, float eps, int64_t rows_per_block) {
  extern __shared__ float lds[];  // [ROPE_WAVES][2*dh]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = dh / 2;
  const int64_t width = (int64_t)(nq + 2 * nkv) * dh;
  float wqa[ROPE_MAX_T], wqb[ROPE_MAX_T], wka[ROPE_MAX_T], wkb[ROPE_MAX_T];
  float gqa[ROPE_MAX_T], gqb[ROPE_MAX_T], gka[ROPE_MAX_T], gkb[ROPE_MAX_T];
#pragma unroll
  for (int t = 0; t < ROPE_MAX_T; ++t) {
    const int i = lane + 64 * t;
    gqa[t] = gqb[t] = gka[t] = gkb[t] = 0.f;
    wqa[t] = wqb[t] = wka[t] = wkb[t] = 0.f;
    if (i < half) {
      wqa[t] = Elem<T>::load(wq, i); wqb[t] = Elem<T>::load(wq, i + half);
      wka[t] = Elem<T>::load(wk, i); wkb[t] = Elem<T>::load(wk, i + half);
    }
  }
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  for (int64_t row = r0 + wave; row < r0 + rows_per_block && row < rows; row += ROPE_WAVES) {
    float csa[ROPE_MAX_T], csb[ROPE_MAX_T], sna[ROPE_MAX_T], snb[ROPE_MAX_T];
#pragma unroll
    for (int t = 0; t < ROPE_MAX_T; ++t) {
      const int i = lane + 64 * t;
      csa[t] = csb[t] = sna[t] = snb[t] = 0.f;
      if (i < half)
        rope_pair<T, TAB>(positions, inv_freq, cos_tab, sin_tab, row, i, dh, csa[t], csb[t],
                          sna[t], snb[t]);
    }
    for (int head = 0; head < nq + nkv; ++head) {
      const bool is_q = head < nq;
      const T* x = qkv + row * width + head * dh;
      const T* g = is_q ? dq + (row * nq + head) * dh : dk + (row * nkv + head - nq) * dh;
      float xa[ROPE_MAX_T], xb[ROPE_MAX_T], ta[ROPE_MAX_T], tb[ROPE_MAX_T];
      float ss = 0.f, s = 0.f;
#pragma unroll
      for (int t = 0; t < ROPE_MAX_T; ++t) {
        const int i = lane + 64 * t;
        xa[t] = xb[t] = ta[t] = tb[t] = 0.f;
        if (i < half) {
          xa[t] = Elem<T>::load(x, i);
          xb[t] = Elem<T>::load(x, i + half);
          const float go = Elem<T>::load(g, i), gh = Elem<T>::load(g, i + half);
          ta[t] = go * csa[t] + gh * snb[t];   // d/d t[i]
          tb[t] = gh * csb[t] - go * sna[t];   // d/d t[i + half]
          ss += xa[t] * xa[t] + xb[t] * xb[t];
          s += ta[t] * (is_q ? wqa[t] : wka[t]) * xa[t] + tb[t] * (is_q ? wqb[t] : wkb[t]) * xb[t];
        }
      }
      ss = wave_sum(ss);
      s = wave_sum(s);
      const float r = 1.0f / sqrtf(ss / (float)dh + eps);
      const float k = s * r * r * r / (float)dh;
      T* out = dqkv + row * width + head * dh;
#pragma unroll
      for (int t = 0; t < ROPE_MAX_T; ++t) {
        const int i = lane + 64 * t;
        if (i < half) {
          const float na = Elem<T>::round(xa[t] * r), nb = Elem<T>::round(xb[t] * r);
          if (is_q) { gqa[t] += ta[t] * na; gqb[t] += tb[t] * nb; }
          else { gka[t] += ta[t] * na; gkb[t] += tb[t] * nb; }
          Elem<T>::store(out, i, r * ta[t] * (is_q ? wqa[t] : wka[t]) - xa[t] * k);
          Elem<T>::store(out, i + half, r * tb[t] * (is_q ? wqb[t] : wkb[t]) - xb[t] * k);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < ROPE_MAX_T; ++t) {
    const int i = lane + 64 * t;
    if (i < half) {
      float* L = lds + wave * 2 * dh;
      L[i] = gqa[t]; L[i + half] = gqb[t];
      L[dh + i] = gka[t]; L[dh + i + half] = gkb[t];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < 2 * dh; c += 64 * ROPE_WAVES) {
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < ROPE_WAVES; ++v) acc += lds[v * 2 * dh + c];
    partial[(int64_t)blockIdx.x * 2 * dh + c] = acc;
  }
}

// ---------------------------------------------------------------------------
// head_dim 128, bf16.  Same arithmetic and rounding points as the kernels
// above.  The 64 rotation angles of a row are computed once per row, one per
// lane (lane l: frequency l), and handed to the lanes that use them by
// shuffles.
//  * forward: eight heads per wavefront pass, 8 lanes per head, lane j owning
//    rotary elements i = 8j..8j+7 and i + 64 (16-byte accesses; 71.6 against
//    85.6 us per 1.7B call with 16 lanes per head and 8-byte accesses);
//  * backward: four heads per pass, 16 lanes per head, lane j owning
//    i = 4j..4j+3 and i + 64 (8-byte accesses: the 8-lane form needs 149
//    VGPRs, 3 wavefronts per SIMD, and ran 139 against 121 us).
// Sums over a head are 8- or 16-lane reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sum16(float v) {
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void load4(const bf16_t* p, float* v) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  v[0] = bf16_to_float((bf16_t)(u.x & 0xffff)); v[1] = bf16_to_float((bf16_t)(u.x >> 16));
  v[2] = bf16_to_float((bf16_t)(u.y & 0xffff)); v[3] = bf16_to_float((bf16_t)(u.y >> 16));
}
__device__ __forceinline__ void store4(bf16_t* p, const float* v) {
  *reinterpret_cast<uint2*>(p) =
      make_uint2(pack_bf16x2(v[0], v[1]),
                 pack_bf16x2(v[2], v[3]));
}

__device__ __forceinline__ float sum8(float v) {
#pragma unroll
  for (int off = 4; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ void __launch_bounds__(64 * ROPE_WAVES)
qknorm_rope128_fwd_kernel(const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ wq,
                          const bf16_t* __restrict__ wk, const int64_t* __restrict__ positions,
                          const float* __restrict__ inv_freq, bf16_t* __restrict__ q_out,
                          bf16_t* __restrict__ k_out, int64_t rows, int nq, int nkv, float eps) {
  const int lane = threadIdx.x & 63, slot = lane >> 3, j = lane & 7;
  const int64_t row = (int64_t)blockIdx.x * ROPE_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int i0 = 8 * j;
  const float pos = (float)positions[row];
  // lane l computes the rotation of frequency l; lane j of a head takes
  // frequencies 8j..8j+7 from lanes 8j..8j+7
  float cs[8], sn[8], wqa[8], wqb[8], wka[8], wkb[8];
  {
    const float ang = pos * inv_freq[lane];
    const float c1 = round_bf16(cosf(ang)), s1 = round_bf16(sinf(ang));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cs[e] = __shfl(c1, i0 + e, 64);
      sn[e] = __shfl(s1, i0 + e, 64);
    }
  }
  Vec8<bf16_t>::load(wq + i0, wqa); Vec8<bf16_t>::load(wq + i0 + 64, wqb);
  Vec8<bf16_t>::load(wk + i0, wka); Vec8<bf16_t>::load(wk + i0 + 64, wkb);
  const int heads = nq + nkv;
  const bf16_t* src = qkv + row * (int64_t)(nq + 2 * nkv) * 128;
  for (int h0 = 0; h0 < heads; h0 += 8) {
    const int head = h0 + slot;
    const bool live = head < heads;
    const bool is_q = head < nq;
    float xa[8], xb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) xa[e] = xb[e] = 0.f;
    if (live) { Vec8<bf16_t>::load(src + head * 128 + i0, xa); Vec8<bf16_t>::load(src + head * 128 + i0 + 64, xb); }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += xa[e] * xa[e] + xb[e] * xb[e];
    ss = sum8(ss);
    const float r = 1.0f / sqrtf(ss / 128.f + eps);
    float oa[8], ob[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = round_bf16((is_q ? wqa[e] : wka[e]) * round_bf16(xa[e] * r));
      const float b = round_bf16((is_q ? wqb[e] : wkb[e]) * round_bf16(xb[e] * r));
      oa[e] = round_bf16(a * cs[e]) + round_bf16(-b * sn[e]);
      ob[e] = round_bf16(b * cs[e]) + round_bf16(a * sn[e]);
    }
    if (live) {
      bf16_t* dst = is_q ? q_out + (row * nq + head) * 128 : k_out + (row * nkv + head - nq) * 128;
      Vec8<bf16_t>::store(dst + i0, oa);
      Vec8<bf16_t>::store(dst + i0 + 64, ob);
    }
  }
}

__global__ void __launch_bounds__(64 * ROPE_WAVES)
qknorm_rope128_bwd_kernel(const bf16_t* __restrict__ dq, const bf16_t* __restrict__ dk,
                          const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ wq,
                          const bf16_t* __restrict__ wk, const int64_t* __restrict__ positions,
                          const float* __restrict__ inv_freq, bf16_t* __restrict__ dqkv,
                          float* __restrict__ partial, int64_t rows, int nq, int nkv, float eps,
                          int64_t rows_per_block) {
  __shared__ float lds[ROPE_WAVES * 4][2 * 128];  // [wave*4 + slot][dwq | dwk]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, slot = lane >> 4, j = lane & 15;
  const int i0 = 4 * j;
  const int64_t width = (int64_t)(nq + 2 * nkv) * 128;
  const float freq = inv_freq[lane];
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  float* L = lds[wave * 4 + slot];
  // the q heads of the block's rows, then the k heads: one weight-gradient
  // accumulator set per lane at a time
#pragma unroll 1
  for (int kind = 0; kind < 2; ++kind) {
    const int h_beg = kind ? nq : 0, h_end = kind ? nq + nkv : nq;
    const bf16_t* w = kind ? wk : wq;
    float wa[4], wb[4], ga[4] = {0.f, 0.f, 0.f, 0.f}, gb[4] = {0.f, 0.f, 0.f, 0.f};
    load4(w + i0, wa); load4(w + i0 + 64, wb);
    for (int64_t row = r0 + wave; row < r0 + rows_per_block && row < rows; row += ROPE_WAVES) {
      // lane l computes the rotation of frequency l; lane j of a head takes
      // frequencies 4j..4j+3 from lanes 4j..4j+3
      float cs[4], sn[4];
      {
        const float ang = (float)positions[row] * freq;
        const float c1 = round_bf16(cosf(ang)), s1 = round_bf16(sinf(ang));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cs[e] = __shfl(c1, i0 + e, 64);
          sn[e] = __shfl(s1, i0 + e, 64);
        }
      }
      for (int h0 = h_beg; h0 < h_end; h0 += 4) {
        const int head = h0 + slot;
        const bool live = head < h_end;
        float xa[4] = {0.f, 0.f, 0.f, 0.f}, xb[4] = {0.f, 0.f, 0.f, 0.f};
        float go[4] = {0.f, 0.f, 0.f, 0.f}, gh[4] = {0.f, 0.f, 0.f, 0.f};
        if (live) {
          const bf16_t* x = qkv + row * width + head * 128;
          const bf16_t* g = kind ? dk + (row * nkv + head - nq) * 128 : dq + (row * nq + head) * 128;
          load4(x + i0, xa); load4(x + i0 + 64, xb);
          load4(g + i0, go); load4(g + i0 + 64, gh);
        }
        float ta[4], tb[4], ss = 0.f, s = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ta[e] = go[e] * cs[e] + gh[e] * sn[e];   // d/d t[i]
          tb[e] = gh[e] * cs[e] - go[e] * sn[e];   // d/d t[i + half]
          ss += xa[e] * xa[e] + xb[e] * xb[e];
          s += ta[e] * wa[e] * xa[e] + tb[e] * wb[e] * xb[e];
        }
        ss = sum16(ss);
        s = sum16(s);
        const float r = 1.0f / sqrtf(ss / 128.f + eps);
        const float k = s * r * r * r / 128.f;
        float oa[4], ob[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ga[e] += ta[e] * round_bf16(xa[e] * r);
          gb[e] += tb[e] * round_bf16(xb[e] * r);
          oa[e] = r * ta[e] * wa[e] - xa[e] * k;
          ob[e] = r * tb[e] * wb[e] - xb[e] * k;
        }
        if (live) {
          bf16_t* out = dqkv + row * width + head * 128;
          store4(out + i0, oa);
          store4(out + i0 + 64, ob);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      L[kind * 128 + i0 + e] = ga[e];
      L[kind * 128 + i0 + 64 + e] = gb[e];
    }
  }
  __syncthreads();
  {
    const int c = threadIdx.x;  // 256 threads = 2 * 128 columns
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < ROPE_WAVES * 4; ++v) acc += lds[v][c];
    partial[(int64_t)blockIdx.x * 256 + c] = acc;
  }
}

// The head_dim-128 backward makes 8-byte accesses, the forward 16-byte ones.
static bool rope128_aligned(const void* a, const void* b, const void* c) {
  return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
           reinterpret_cast<uintptr_t>(c)) & 7) == 0;
}

static bool rope128_aligned16(const void* a, const void* b, const void* c) {
  return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
           reinterpret_cast<uintptr_t>(c)) & 15) == 0;
}

static int check_rope(int64_t rows, int64_t nq, int64_t nkv, int64_t dh) {
  ALODLM_CHECK_ARG(rows >= 0 && nq > 0 && nkv > 0, "qknorm_rope: bad head counts");
  ALODLM_CHECK_ARG(dh > 0 && dh % 2 == 0 && dh <= 128 * ROPE_MAX_T,
                   "qknorm_rope: head_dim must be even and <= %d", 128 * ROPE_MAX_T);
  return ALODLM_OK;
}

extern "C" int alodlm_qknorm_rope_fwd(const void* qkv, const void* wq, const void* wk,
                                      const int64_t* positions, const float* inv_freq, void* q_out,
                                      void* k_out, int64_t rows, int64_t nq, int64_t nkv,
                                      int64_t dh, float eps, int dtype, void* stream) {
  int rc = check_rope(rows, nq, nkv, dh);
  if (rc) return rc;
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    if (std::is_same<T, bf16_t>::value && dh == 128 && rope128_aligned16(qkv, q_out, k_out) &&
        rope128_aligned16(wq, wk, wk)) {
      qknorm_rope128_fwd_kernel<<<ceil_div_u(rows, ROPE_WAVES), 64 * ROPE_WAVES, 0,
                                  as_stream(stream)>>>(
          (const bf16_t*)qkv, (const bf16_t*)wq, (const bf16_t*)wk, positions, inv_freq,
          (bf16_t*)q_out, (bf16_t*)k_out, rows, (int)nq, (int)nkv, eps);
      break;
    }
    qknorm_rope_fwd_kernel<T, false><<<ceil_div_u(rows, ROPE_WAVES), 64 * ROPE_WAVES, 0,
                                       as_stream(stream)>>>(
        (const T*)qkv, (const T*)wq, (const T*)wk, positions, inv_freq, nullptr, nullptr,
        (T*)q_out, (T*)k_out, rows, (int)nq, (int)nkv, (int)dh, eps);
  });
  ALODLM_CHECK_LAUNCH("qknorm_rope_fwd");
  return ALODLM_OK;
}

extern "C" int64_t alodlm_qknorm_rope_bwd_workspace(int64_t rows, int64_t nq, int64_t nkv,
                                                    int64_t dh) {
  (void)nq; (void)nkv;
  // per-block partial rows [dwq | dwk], then the column reduction's group sums
  const int64_t rpb = bwd_rows_per_block(rows);
  return ((rows + rpb - 1) / rpb) * 2 * dh + COLUMN_REDUCE_MAX_GROUPS * dh;
}

extern "C" int alodlm_qknorm_rope_bwd(const void* dq, const void* dk, const void* qkv,
                                      const void* wq, const void* wk, const int64_t* positions,
                                      const float* inv_freq, void* dqkv, float* dwq_accum,
                                      float* dwk_accum, float* workspace, int64_t rows, int64_t nq,
                                      int64_t nkv, int64_t dh, float eps, int dtype, void* stream) {
  int rc = check_rope(rows, nq, nkv, dh);
  if (rc) return rc;
  if (rows == 0) return ALODLM_OK;
  const int64_t rpb = bwd_rows_per_block(rows);
  const int64_t nparts = (rows + rpb - 1) / rpb;
  hipStream_t st = as_stream(stream);
  ALODLM_DISPATCH(dtype, T, {
    if (std::is_same<T, bf16_t>::value && dh == 128 && rope128_aligned(dq, dk, qkv) &&
        rope128_aligned(dqkv, wq, wk)) {
      qknorm_rope128_bwd_kernel<<<(unsigned)nparts, 64 * ROPE_WAVES, 0, st>>>(
          (const bf16_t*)dq, (const bf16_t*)dk, (const bf16_t*)qkv, (const bf16_t*)wq,
          (const bf16_t*)wk, positions, inv_freq, (bf16_t*)dqkv, workspace, rows, (int)nq,
          (int)nkv, eps, rpb);
      break;
    }
    qknorm_rope_bwd_kernel<T, false><<<(unsigned)nparts, 64 * ROPE_WAVES,
                                       ROPE_WAVES * 2 * dh * sizeof(float), st>>>(
        (const T*)dq, (const T*)dk, (const T*)qkv, (const T*)wq, (const T*)wk, positions,
        inv_freq, nullptr, nullptr, (T*)dqkv, workspace, rows, (int)nq, (int)nkv, (int)dh, eps,
        rpb);
  });
  ALODLM_CHECK_LAUNCH("qknorm_rope_bwd");
  float* tmp = workspace + nparts * 2 * dh;
  rc = column_reduce(workspace, nparts, 2 * dh, 0, dh, dwq_accum, tmp, st);
  if (rc) return rc;
  return column_reduce(workspace, nparts, 2 * dh, dh, dh, dwk_accum, tmp, st);
}

// ---------------------------------------------------------------------------
// Table-driven forms (alodlm/model.py:41-46 takes cos/sin tables [rows, dh]):
// q/k norm + rotary on the projections, and the rotary alone.
// ---------------------------------------------------------------------------
extern "C" int alodlm_qknorm_rotary_fwd(const void* qkv, const void* wq, const void* wk,
                                        const void* cos_tab, const void* sin_tab, void* q_out,
                                        void* k_out, int64_t rows, int64_t nq, int64_t nkv,
                                        int64_t dh, float eps, int dtype, void* stream) {
  int rc = check_rope(rows, nq, nkv, dh);
  if (rc) return rc;
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    qknorm_rope_fwd_kernel<T, true><<<ceil_div_u(rows, ROPE_WAVES), 64 * ROPE_WAVES, 0,
                                      as_stream(stream)>>>(
        (const T*)qkv, (const T*)wq, (const T*)wk, nullptr, nullptr, (const T*)cos_tab,
        (const T*)sin_tab, (T*)q_out, (T*)k_out, rows, (int)nq, (int)nkv, (int)dh, eps);
  });
  ALODLM_CHECK_LAUNCH("qknorm_rotary_fwd");
  return ALODLM_OK;
}

extern "C" int alodlm_qknorm_rotary_bwd(const void* dq, const void* dk, const void* qkv,
                                        const void* wq, const void* wk, const void* cos_tab,
                                        const void* sin_tab, void* dqkv, float* dwq_accum,
                                        float* dwk_accum, float* workspace, int64_t rows,
                                        int64_t nq, int64_t nkv, int64_t dh, float eps, int dtype,
                                        void* stream) {
  int rc = check_rope(rows, nq, nkv, dh);
  if (rc) return rc;
  if (rows == 0) return ALODLM_OK;
  const int64_t rpb = bwd_rows_per_block(rows);
  const int64_t nparts = (rows + rpb - 1) / rpb;
  hipStream_t st = as_stream(stream);
  ALODLM_DISPATCH(dtype, T, {
    qknorm_rope_bwd_kernel<T, true><<<(unsigned)nparts, 64 * ROPE_WAVES,
                                      ROPE_WAVES * 2 * dh * sizeof(float), st>>>(
        (const T*)dq, (const T*)dk, (const T*)qkv, (const T*)wq, (const T*)wk, nullptr, nullptr,
        (const T*)cos_tab, (const T*)sin_tab, (T*)dqkv, workspace, rows, (int)nq, (int)nkv,
        (int)dh, eps, rpb);
  });
  ALODLM_CHECK_LAUNCH("qknorm_rotary_bwd");
  float* tmp = workspace + nparts * 2 * dh;
  rc = column_reduce(workspace, nparts, 2 * dh, 0, dh, dwq_accum, tmp, st);
  if (rc) return rc;
  return column_reduce(workspace, nparts, 2 * dh, dh, dh, dwk_accum, tmp, st);
}

// out = x * cos + rotate_half(x) * sin for every head of a row, with the
// reference's three roundings (product, product, sum); BWD applies the
// transpose: dx[i] = dy[i] cos[i] + dy[i+h] sin[i+h],
// dx[i+h] = dy[i+h] cos[i+h] - dy[i] sin[i], each product rounded and the
// sum rounded, as the reference's bf16 autograd accumulates them (float32:
// every product and the sum rounded once, no contraction).
template <typename T, bool BWD>
__global__ void __launch_bounds__(256)
rotary_kernel(const T* __restrict__ x, const T* __restrict__ cos_tab,
              const T* __restrict__ sin_tab, T* __restrict__ out, int64_t rows, int heads,
              int dh) {
  // products and sums stay separately rounded, as the reference evaluates
  // them (no fused multiply-add)
#pragma clang fp contract(off)
  const int half = dh / 2;
  const int64_t n = rows * heads * half;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(e % half);
    const int64_t rh = e / half;          // row * heads + head
    const int64_t row = rh / heads;
    const float a = Elem<T>::load(x, rh * dh + i), b = Elem<T>::load(x, rh * dh + i + half);
    const float ca = Elem<T>::load(cos_tab, row * dh + i);
    const float cb = Elem<T>::load(cos_tab, row * dh + i + half);
    const float sa = Elem<T>::load(sin_tab, row * dh + i);
    const float sb = Elem<T>::load(sin_tab, row * dh + i + half);
    float lo, hi;
    if (BWD) {
      lo = Elem<T>::round(a * ca) + Elem<T>::round(b * sb);
      hi = Elem<T>::round(b * cb) + Elem<T>::round(-a * sa);
    } else {
      lo = Elem<T>::round(a * ca) + Elem<T>::round(-b * sa);
      hi = Elem<T>::round(b * cb) + Elem<T>::round(a * sb);
    }
    Elem<T>::store(out, rh * dh + i, lo);
    Elem<T>::store(out, rh * dh + i + half, hi);
  }
}

static int rotary_launch(const void* x, const void* cos_tab, const void* sin_tab, void* out,
                         int64_t rows, int64_t heads, int64_t dh, int dtype, bool bwd,
                         hipStream_t st) {
  ALODLM_CHECK_ARG(rows >= 0 && heads > 0 && dh > 0 && dh % 2 == 0,
                   "rotary: head_dim must be even and the head count positive");
  if (rows == 0) return ALODLM_OK;
  const int64_t n = rows * heads * (dh / 2);
  const unsigned grid = (unsigned)(n / 256 + 1 < 65536 ? n / 256 + 1 : 65536);
  ALODLM_DISPATCH(dtype, T, {
    if (bwd)
      rotary_kernel<T, true><<<grid, 256, 0, st>>>((const T*)x, (const T*)cos_tab,
                                                   (const T*)sin_tab, (T*)out, rows, (int)heads,
                                                   (int)dh);
    else
      rotary_kernel<T, false><<<grid, 256, 0, st>>>((const T*)x, (const T*)cos_tab,
                                                    (const T*)sin_tab, (T*)out, rows, (int)heads,
                                                    (int)dh);
  });
  ALODLM_CHECK_LAUNCH("rotary");
  return ALODLM_OK;
}

extern "C" int alodlm_rotary_fwd(const void* x, const void* cos_tab, const void* sin_tab,
                                 void* out, int64_t rows, int64_t heads, int64_t dh, int dtype,
                                 void* stream) {
  return rotary_launch(x, cos_tab, sin_tab, out, rows, heads, dh, dtype, false,
                       as_stream(stream));
}

extern "C" int alodlm_rotary_bwd(const void* dout, const void* cos_tab, const void* sin_tab,
                                 void* dx, int64_t rows, int64_t heads, int64_t dh, int dtype,
                                 void* stream) {
  return rotary_launch(dout, cos_tab, sin_tab, dx, rows, heads, dh, dtype, true,
                       as_stream(stream));
}
