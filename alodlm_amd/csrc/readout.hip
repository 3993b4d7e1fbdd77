// Readout side of each recurrent depth: the final norm fused with the gate
// head, the carry norm fused with re-embedding, exit sampling, the selection
// of loss-bearing rows, and the vocabulary cross-entropy.
#include "common.h"

#define RO_WAVES 4

// readout = norm(x); gate = cast(cast(readout.w + b) + depth_bias[d])
// (alodlm/model.py:160-162 and GateHead.forward :37-38).
template <typename T>
__global__ void __launch_bounds__(64 * RO_WAVES)
final_norm_gate_kernel(const T* __restrict__ x, const T* __restrict__ wf, const T* __restrict__ gw,
                       const T* __restrict__ gb, const T* __restrict__ db, int64_t depth,
                       T* __restrict__ readout, float* __restrict__ rstd, float* __restrict__ gate,
                       int64_t rows, int64_t H, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * RO_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * H;
  T* yr = readout + row * H;
  float ss = 0.f;
  for (int64_t c = lane; c < H; c += 64) {
    float v = Elem<T>::load(xr, c);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  float dot = 0.f;
  for (int64_t c = lane; c < H; c += 64) {
    float y = Elem<T>::round(Elem<T>::load(wf, c) * Elem<T>::round(Elem<T>::load(xr, c) * r));
    Elem<T>::store(yr, c, y);
    dot += y * Elem<T>::load(gw, c);
  }
  dot = wave_sum(dot);
  if (lane == 0) {
    rstd[row] = r;
    float g = Elem<T>::round(dot + Elem<T>::load(gb, 0));
    gate[row] = Elem<T>::round(g + Elem<T>::load(db, depth));
  }
}

// out = exits <= d ? table[original] : norm(x)   (model.py:153-154,168)
template <typename T>
__global__ void __launch_bounds__(64 * RO_WAVES)
carry_select_kernel(const T* __restrict__ x, const T* __restrict__ wf, const T* __restrict__ table,
                    const int64_t* __restrict__ original, const int32_t* __restrict__ exits,
                    int64_t depth, T* __restrict__ out, float* __restrict__ rstd, int64_t rows,
                    int64_t H, float eps, int64_t vocab) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * RO_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * H;
  T* yr = out + row * H;
  float ss = 0.f;
  for (int64_t c = lane; c < H; c += 64) {
    float v = Elem<T>::load(xr, c);
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (lane == 0) rstd[row] = r;
  if (exits[row] <= depth) {
    const int64_t id = original[row];
    if (id < 0 || id >= vocab) {
      for (int64_t c = lane; c < H; c += 64) Elem<T>::store(yr, c, NAN);
    } else {
      const T* er = table + id * H;
      for (int64_t c = lane; c < H; c += 64) yr[c] = er[c];
    }
  } else {
    for (int64_t c = lane; c < H; c += 64)
      Elem<T>::store(yr, c, Elem<T>::load(wf, c) * Elem<T>::round(Elem<T>::load(xr, c) * r));
  }
}

__global__ void exit_update_kernel(const float* __restrict__ gate, const float* __restrict__ u,
                                   const uint8_t* __restrict__ masked, int32_t* __restrict__ exits,
                                   int32_t depth, int32_t K, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float hazard = sigmoidf_ref(gate[r]);
  if (u[r] < hazard && masked[r] && exits[r] == K) exits[r] = depth + 1;
}

__global__ void __launch_bounds__(1024)
inverse_weight_sum_kernel(const uint8_t* __restrict__ masked, const float* __restrict__ p,
                          int64_t rows, float* __restrict__ out) {
  __shared__ float scratch[16];
  float s = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x)
    if (masked[r]) s += 1.0f / (p[r] + 1e-8f);
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) out[0] = s;
}

// Stable compaction of the loss-bearing rows of depth d with their targets and
// dL/dce coefficients (loss.py:55-61 for masked rows; loss.py:12-32 and
// model.py:183-185 for the autoregressive rows).
__global__ void __launch_bounds__(1024)
select_rows_kernel(const uint8_t* __restrict__ masked, const int32_t* __restrict__ exits,
                   const int64_t* __restrict__ original, const int32_t* __restrict__ ar_target,
                   const float* __restrict__ gates, const float* __restrict__ mask_prob,
                   const float* __restrict__ wsum, float ar_coef, int32_t depth, int32_t K,
                   int64_t rows, int32_t* __restrict__ sel_rows, int32_t* __restrict__ sel_target,
                   float* __restrict__ sel_coef, int32_t* __restrict__ sel_count) {
  __shared__ int32_t wave_counts[16];
  __shared__ int32_t base;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  if (threadIdx.x == 0) base = 0;
  __syncthreads();
  const float inv_wsum = 1.0f / wsum[0];
  for (int64_t start = 0; start < rows; start += blockDim.x) {
    const int64_t r = start + threadIdx.x;
    int take = 0, target = -1;
    float coef = 0.f;
    if (r < rows) {
      if (masked[r] && exits[r] > depth) {
        take = 1;
        target = (int)original[r];
        float log_surv = 0.f;
        for (int j = 0; j < depth; ++j) log_surv -= softplusf(gates[(int64_t)j * rows + r]);
        const bool last = exits[r] == depth + 1 || depth == K - 1;
        const float log_stick =
            last ? log_surv : log_surv - softplusf(-gates[(int64_t)depth * rows + r]);
        const float w = (1.0f / (mask_prob[r] + 1e-8f)) * inv_wsum;
        coef = 0.5f * w * expf(log_stick);
      } else if (ar_target[r] >= 0) {
        take = 1;
        target = ar_target[r];
        coef = ar_coef;
      }
    }
    const uint64_t ballot = __ballot(take);
    const int prefix = __popcll(ballot & ((1ull << lane) - 1ull));
    if (lane == 0) wave_counts[wave] = __popcll(ballot);
    __syncthreads();
    int offset = base;
    for (int w = 0; w < wave; ++w) offset += wave_counts[w];
    if (take) {
      sel_rows[offset + prefix] = (int32_t)r;
      sel_target[offset + prefix] = target;
      sel_coef[offset + prefix] = coef;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int total = 0;
      for (int w = 0; w < nwaves; ++w) total += wave_counts[w];
      base += total;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) sel_count[0] = base;
}

template <typename T>
__global__ void gather_rows_kernel(const T* __restrict__ src, const int32_t* __restrict__ sel,
                                   int64_t n, T* __restrict__ dst, int64_t H) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * H) return;
  const int64_t j = i / H, c = i % H;
  dst[i] = src[(int64_t)sel[j] * H + c];
}

template <typename T>
__global__ void zero_kernel(T* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = (T)0;
}

template <typename T>
__global__ void scatter_rows_kernel(const T* __restrict__ src, const int32_t* __restrict__ sel,
                                    int64_t n, T* __restrict__ dst, int64_t H) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * H) return;
  const int64_t j = i / H, c = i % H;
  dst[(int64_t)sel[j] * H + c] = src[i];
}

// The same row moves in 16-byte units (rows of a whole number of units,
// 16-byte aligned buffers): grid x covers a row's U units, grid y rows
// j0 + y; SCATTER: dst row sel[j] <- src row j, else dst row j <- src row
// sel[j].
template <bool SCATTER>
__global__ void move_rows16_kernel(const uint4* __restrict__ src, const int32_t* __restrict__ sel,
                                   int64_t j0, uint4* __restrict__ dst, int64_t U) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= U) return;
  const int64_t j = j0 + blockIdx.y;
  const int64_t other = sel[j];
  if (SCATTER) dst[other * U + u] = src[j * U + u];
  else dst[j * U + u] = src[other * U + u];
}

__global__ void zero16_kernel(uint4* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = make_uint4(0u, 0u, 0u, 0u);
}

// rows of 16-byte units: launches of at most 65535 rows
template <bool SCATTER>
static void move_rows16(const void* src, const int32_t* sel, int64_t n, void* dst, int64_t U,
                        hipStream_t st) {
  const unsigned threads = (unsigned)(U < 256 ? (U + 63) / 64 * 64 : 256);
  for (int64_t j0 = 0; j0 < n; j0 += 65535) {
    const int64_t m = n - j0 < 65535 ? n - j0 : 65535;
    move_rows16_kernel<SCATTER><<<dim3(ceil_div_u(U, threads), (unsigned)m), threads, 0, st>>>(
        (const uint4*)src, sel, j0, (uint4*)dst, U);
  }
}

static bool rows16(const void* a, const void* b, int64_t row_bytes) {
  return row_bytes % 16 == 0 &&
         ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
}

#define CE_LOG2E 1.4426950408889634f

// ce = lse - logit[target] (rounded like the reference's CE output),
// entropy = lse - sum p*logit, logits <- coef*(softmax - onehot).  float
// logits keep expf throughout; bf16 logits take the exp2 path.
template <typename T, bool V8>
__global__ void __launch_bounds__(256)
cross_entropy_kernel(T* __restrict__ logits, const int32_t* __restrict__ target,
                     const float* __restrict__ coef, const int32_t* __restrict__ n_rows,
                     int64_t V, float* __restrict__ ce, float* __restrict__ entropy) {
  constexpr bool FAST = sizeof(T) == 2;
  __shared__ float sm[4], ss[4], st[4];
  const int64_t row = blockIdx.x;
  if (row >= n_rows[0]) return;
  T* lr = logits + row * V;
  float m = -INFINITY, s = 0.f, t = 0.f;
  auto add = [&](float x) {
    if (x > m) {
      const float scale = expf(m - x);
      s = s * scale + 1.f;
      t = t * scale + x;
      m = x;
    } else {
      const float e = expf(x - m);
      s += e;
      t += e * x;
    }
  };
  if (V8 && FAST) {
    // bf16 logits: one rescale per 8 values and the hardware exp2 (its error,
    // a few float ulps, is far below the bf16 rounding of every output)
    for (int64_t c = (int64_t)threadIdx.x * 8; c < V; c += 256 * 8) {
      float v[8];
      Vec8<T>::load(lr + c, v);
      float cm = v[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) cm = fmaxf(cm, v[i]);
      if (cm > m) {
        const float scale = __builtin_amdgcn_exp2f((m - cm) * CE_LOG2E);  // 0 when m = -inf
        s *= scale;
        t *= scale;
        m = cm;
      }
      const float m2 = m * CE_LOG2E;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(v[i], CE_LOG2E, -m2));
        s += e;
        t = fmaf(e, v[i], t);
      }
    }
  } else if (V8) {
    for (int64_t c = (int64_t)threadIdx.x * 8; c < V; c += 256 * 8) {
      float v[8];
      Vec8<T>::load(lr + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) add(v[i]);
    }
  } else {
    for (int64_t c = threadIdx.x; c < V; c += 256) add(Elem<T>::load(lr, c));
  }
  // combine (m, s, t) across the block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float M = wave_max(m);
  float scale = (m == -INFINITY) ? 0.f : expf(m - M);
  float S = wave_sum(s * scale), Tt = wave_sum(t * scale);
  if (lane == 0) { sm[wave] = M; ss[wave] = S; st[wave] = Tt; }
  __syncthreads();
  float gm = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
  float gs = 0.f, gt = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float f = (sm[w] == -INFINITY) ? 0.f : expf(sm[w] - gm);
    gs += ss[w] * f;
    gt += st[w] * f;
  }
  const float lse = gm + logf(gs);
  int tg = target[row];
  const float cf = coef[row];
  const bool valid = tg >= 0 && tg < V;  // an out-of-range target yields NaN, never a read
  if (threadIdx.x == 0) {
    const float xt = valid ? Elem<T>::load(lr, tg) : NAN;
    ce[row] = Elem<T>::round(lse - xt);
    if (entropy) entropy[row] = lse - gt / gs;
  }
  if (!valid) tg = -1;
  __syncthreads();  // the target logit is read above before it is overwritten
  if (V8 && FAST) {
    const float lse2 = lse * CE_LOG2E;
    for (int64_t c = (int64_t)threadIdx.x * 8; c < V; c += 256 * 8) {
      float v[8];
      Vec8<T>::load(lr + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = cf * (__builtin_amdgcn_exp2f(fmaf(v[i], CE_LOG2E, -lse2)) - (c + i == tg ? 1.f : 0.f));
      Vec8<T>::store(lr + c, v);
    }
  } else if (V8) {
    for (int64_t c = (int64_t)threadIdx.x * 8; c < V; c += 256 * 8) {
      float v[8];
      Vec8<T>::load(lr + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = cf * (expf(v[i] - lse) - (c + i == tg ? 1.f : 0.f));
      Vec8<T>::store(lr + c, v);
    }
  } else {
    for (int64_t c = threadIdx.x; c < V; c += 256) {
      const float v = Elem<T>::load(lr, c);
      Elem<T>::store(lr, c, cf * (expf(v - lse) - (c == tg ? 1.f : 0.f)));
    }
  }
}

// The same for bf16 rows of at most 8 * CE_THREADS * NCH logits held in the
// registers of CE_THREADS threads (up to 128 VGPRs each): each row is read from
// memory once and written once (the two-pass kernel above reads it twice, and
// a row of a large vocabulary does not stay in L2 between the passes).  One
// workgroup per CU walks rows blockIdx.x, blockIdx.x + gridDim.x, ...: as it
// writes chunk j of its current row it loads chunk j of its next row into the
// same registers, so the stream of writes of one row overlaps the reads of
// the next instead of alternating with them.
constexpr int CE_THREADS = 1024;

template <int NCH>
__global__ void __launch_bounds__(CE_THREADS)
cross_entropy_row_kernel(bf16_t* __restrict__ logits, const int32_t* __restrict__ target,
                         const float* __restrict__ coef, const int32_t* __restrict__ n_rows,
                         int64_t V, float* __restrict__ ce, float* __restrict__ entropy) {
  constexpr int NW = CE_THREADS / 64;
  __shared__ float red[2][NW];
  const int64_t rows = n_rows[0];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint4 buf[NCH];
  // 32-bit chunk positions (a row is below 2^31 elements): the compiler then
  // folds j into immediates instead of keeping a 64-bit position per chunk
  const uint32_t Vu = (uint32_t)V, t8 = threadIdx.x * 8u;
  auto first = [&](int j) { return (uint32_t)(j * CE_THREADS * 8) + t8; };
  auto live = [&](int j) { return first(j) < Vu; };
  // Rows are addressed as buffers: one 32-bit lane offset (this thread's
  // 16 bytes of a 16 KB chunk) plus the chunk's byte offset as the scalar
  // offset, so no per-chunk address is kept in vector registers across rows;
  // the range check returns zeros past the row (loads) and drops stores there.
  const uint32_t voff = threadIdx.x * 16u;
  constexpr uint32_t CHUNK = CE_THREADS * 16;
  auto rsrc = [&](int64_t r) {
    return __builtin_amdgcn_make_buffer_rsrc(logits + r * V, 0, (int)(V * 2), 0x00020000);
  };
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  // non-temporal (cache policy 2): a depth's logits are several GB, read
  // once and written once here
  constexpr int NT = 2;
  auto load = [&](__amdgpu_buffer_rsrc_t rs, int j) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, j * CHUNK, NT));
  };
  int64_t row = blockIdx.x;
  if (row >= rows) return;
  {
    const __amdgpu_buffer_rsrc_t rs = rsrc(row);
#pragma unroll
    for (int j = 0; j < NCH; ++j) buf[j] = load(rs, j);
  }
  auto value = [&](int j, int i) {
    const uint32_t w = (&buf[j].x)[i >> 1];
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  };
  for (; row < rows; row += gridDim.x) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(row);
    const int64_t next = row + gridDim.x;
    const __amdgpu_buffer_rsrc_t rn = rsrc(next < rows ? next : row);
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      if (live(j))
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, value(j, i));
    m = wave_max(m);
    // the packed chunks are re-read by each pass: the unpacked float values of
    // one pass are not kept for the next (that would take a register per
    // logit); an empty asm that claims to change them makes sure of it
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      asm volatile("" : "+v"(buf[j].x), "+v"(buf[j].y), "+v"(buf[j].z), "+v"(buf[j].w));
    if (lane == 0) red[0][wave] = m;
    __syncthreads();
    float M = red[0][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, red[0][w]);
    const float m2 = M * CE_LOG2E;
    float s = 0.f, t = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      if (live(j))
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float x = value(j, i);
          const float e = __builtin_amdgcn_exp2f(fmaf(x, CE_LOG2E, -m2));
          s += e;
          t = fmaf(e, x, t);
        }
    s = wave_sum(s);
    t = wave_sum(t);
#pragma unroll
    for (int j = 0; j < NCH; ++j)
      asm volatile("" : "+v"(buf[j].x), "+v"(buf[j].y), "+v"(buf[j].z), "+v"(buf[j].w));
    __syncthreads();  // every wave has read red[0]
    if (lane == 0) { red[0][wave] = s; red[1][wave] = t; }
    __syncthreads();
    float S = 0.f, Tt = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) { S += red[0][w]; Tt += red[1][w]; }
    const float lse = M + logf(S);
    int tg = target[row];
    const float cf = coef[row];
    const bool valid = tg >= 0 && (uint32_t)tg < Vu;  // an out-of-range target yields NaN, never a read
    if (threadIdx.x == 0) {
      const float xt = valid ? bf16_to_float(logits[row * V + tg]) : NAN;
      ce[row] = round_bf16(lse - xt);
      if (entropy) entropy[row] = lse - Tt / S;
    }
    if (!valid) tg = -1;
    // the target logit is read above before it is overwritten, and every wave
    // has read red[] before the next row's reductions write it
    __syncthreads();
    const float lse2 = lse * CE_LOG2E;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const uint32_t c = first(j);
      if (c < Vu) {
        float g[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          g[i] = __builtin_amdgcn_exp2f(fmaf(value(j, i), CE_LOG2E, -lse2));
        if ((uint32_t)tg - c < 8u) {  // the target's chunk (one lane of the row)
#pragma unroll
          for (int i = 0; i < 8; ++i) g[i] -= c + i == (uint32_t)tg ? 1.f : 0.f;
        }
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(cf * g[2 * i], cf * g[2 * i + 1]);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{w[0], w[1], w[2], w[3]}, rs, voff,
                                               j * CHUNK, NT);
      }
      // the next row's chunk j into the registers just freed (the last row
      // re-reads its own chunk, which is never used); the chunks are kept in
      // order, so that no chunk's output is computed early and held
      buf[j] = load(rn, j);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

constexpr int CE_ROW_NCH = 19;  // rows of up to 155648 bf16 logits

__global__ void scatter_ce_kernel(const float* __restrict__ ce, const int32_t* __restrict__ sel,
                                  const int32_t* __restrict__ n_rows, int64_t max_rows,
                                  float* __restrict__ ce_full) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= max_rows || j >= n_rows[0]) return;
  ce_full[sel[j]] = ce[j];
}

// partial[blk, 0:H] = sum_r dgate[r]*readout[r]; partial[blk, H] = sum_r dgate[r]
// over the block's kGateBwdRows rows.  grid.y walks row blocks, grid.x column
// chunks of 8 * 256; each thread keeps 8 column sums in registers and reads
// 16-byte row pieces (rows whose dgate is 0, the unmasked ones, are skipped:
// the test is uniform across the block).
template <typename T, bool V8>
__global__ void __launch_bounds__(256)
gate_bwd_kernel(const float* __restrict__ dgate, const T* __restrict__ readout,
                float* __restrict__ partial, int64_t rows, int64_t H, int64_t rows_per_block) {
  constexpr int W = V8 ? 8 : 1;
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * W;
  const int64_t r0 = (int64_t)blockIdx.y * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float gsum = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float g = dgate[r];
    if (g == 0.f) continue;
    gsum += g;
    if (c < H) {
      float v[8];
      if (V8) Vec8<T>::load(readout + r * H + c, v);
      else v[0] = Elem<T>::load(readout, r * H + c);
#pragma unroll
      for (int e = 0; e < W; ++e) acc[e] += g * v[e];
    }
  }
  float* out = partial + (int64_t)blockIdx.y * (H + 1);
  if (c < H) {
#pragma unroll
    for (int e = 0; e < W; ++e) out[c + e] = acc[e];
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[H] = gsum;
}

__global__ void gate_bwd_reduce_kernel(const float* __restrict__ partial, int64_t nparts, int64_t H,
                                       float scale, float* __restrict__ gw, float* __restrict__ gb,
                                       float* __restrict__ gdb) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c > H) return;
  float s = 0.f;
  for (int64_t p = 0; p < nparts; ++p) s += partial[p * (H + 1) + c];
  s *= scale;
  if (c < H) gw[c] += s;
  else { gb[0] += s; gdb[0] += s; }
}

static const int64_t kGateBwdRows = 64;

extern "C" int alodlm_final_norm_gate(const void* x, const void* wf, const void* gate_w,
                                      const void* gate_b, const void* depth_bias, int64_t depth,
                                      void* readout, float* rstd, float* gate, int64_t rows,
                                      int64_t hidden, float eps, int dtype, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && hidden > 0, "final_norm_gate: bad shape");
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    final_norm_gate_kernel<T><<<ceil_div_u(rows, RO_WAVES), 64 * RO_WAVES, 0, as_stream(stream)>>>(
        (const T*)x, (const T*)wf, (const T*)gate_w, (const T*)gate_b, (const T*)depth_bias,
        depth, (T*)readout, rstd, gate, rows, hidden, eps);
  });
  ALODLM_CHECK_LAUNCH("final_norm_gate");
  return ALODLM_OK;
}

extern "C" int alodlm_carry_select(const void* x, const void* wf, const void* table,
                                   const int64_t* original, const int32_t* exits, int64_t depth,
                                   void* out, float* rstd, int64_t rows, int64_t hidden,
                                   int64_t vocab, float eps, int dtype, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && hidden > 0, "carry_select: bad shape");
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    carry_select_kernel<T><<<ceil_div_u(rows, RO_WAVES), 64 * RO_WAVES, 0, as_stream(stream)>>>(
        (const T*)x, (const T*)wf, (const T*)table, original, exits, depth, (T*)out, rstd, rows,
        hidden, eps, vocab);
  });
  ALODLM_CHECK_LAUNCH("carry_select");
  return ALODLM_OK;
}

extern "C" int alodlm_exit_update(const float* gate, const float* uniforms, const uint8_t* masked,
                                  int32_t* exits, int64_t depth, int64_t max_depth, int64_t rows,
                                  void* stream) {
  ALODLM_CHECK_ARG(depth >= 0 && depth < max_depth - 1, "exit_update: depth out of range");
  if (rows == 0) return ALODLM_OK;
  exit_update_kernel<<<ceil_div_u(rows, 256), 256, 0, as_stream(stream)>>>(
      gate, uniforms, masked, exits, (int32_t)depth, (int32_t)max_depth, rows);
  ALODLM_CHECK_LAUNCH("exit_update");
  return ALODLM_OK;
}

extern "C" int alodlm_inverse_weight_sum(const uint8_t* masked, const float* mask_prob,
                                         int64_t rows, float* wsum, void* stream) {
  inverse_weight_sum_kernel<<<1, 1024, 0, as_stream(stream)>>>(masked, mask_prob, rows, wsum);
  ALODLM_CHECK_LAUNCH("inverse_weight_sum");
  return ALODLM_OK;
}

extern "C" int alodlm_select_rows(const uint8_t* masked, const int32_t* exits,
                                  const int64_t* original, const int32_t* ar_target,
                                  const float* gates, const float* mask_prob, const float* wsum,
                                  float ar_coef, int64_t depth, int64_t max_depth, int64_t rows,
                                  int32_t* sel_rows, int32_t* sel_target, float* sel_coef,
                                  int32_t* sel_count, void* stream) {
  ALODLM_CHECK_ARG(depth >= 0 && depth < max_depth, "select_rows: depth out of range");
  select_rows_kernel<<<1, 1024, 0, as_stream(stream)>>>(
      masked, exits, original, ar_target, gates, mask_prob, wsum, ar_coef, (int32_t)depth,
      (int32_t)max_depth, rows, sel_rows, sel_target, sel_coef, sel_count);
  ALODLM_CHECK_LAUNCH("select_rows");
  return ALODLM_OK;
}

extern "C" int alodlm_gather_rows(const void* src, const int32_t* sel_rows, int64_t n_sel,
                                  void* dst, int64_t hidden, int dtype, void* stream) {
  if (n_sel == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    const int64_t row_bytes = hidden * (int64_t)sizeof(T);
    if (rows16(src, dst, row_bytes))
      move_rows16<false>(src, sel_rows, n_sel, dst, row_bytes / 16, as_stream(stream));
    else
      gather_rows_kernel<T><<<ceil_div_u(n_sel * hidden, 256), 256, 0, as_stream(stream)>>>(
          (const T*)src, sel_rows, n_sel, (T*)dst, hidden);
  });
  ALODLM_CHECK_LAUNCH("gather_rows");
  return ALODLM_OK;
}

extern "C" int alodlm_scatter_rows(const void* src, const int32_t* sel_rows, int64_t n_sel,
                                   void* dst, int64_t rows, int64_t hidden, int dtype,
                                   void* stream) {
  ALODLM_DISPATCH(dtype, T, {
    const int64_t row_bytes = hidden * (int64_t)sizeof(T);
    if (rows16(src, dst, row_bytes)) {
      const int64_t units = rows * row_bytes / 16;
      const int64_t blocks = (units + 255) / 256;
      zero16_kernel<<<(unsigned)(blocks < 8192 ? blocks : 8192), 256, 0, as_stream(stream)>>>(
          (uint4*)dst, units);
      if (n_sel > 0) move_rows16<true>(src, sel_rows, n_sel, dst, row_bytes / 16, as_stream(stream));
    } else {
      zero_kernel<T><<<ceil_div_u(rows * hidden, 256), 256, 0, as_stream(stream)>>>(
          (T*)dst, rows * hidden);
      if (n_sel > 0)
        scatter_rows_kernel<T><<<ceil_div_u(n_sel * hidden, 256), 256, 0, as_stream(stream)>>>(
            (const T*)src, sel_rows, n_sel, (T*)dst, hidden);
    }
  });
  ALODLM_CHECK_LAUNCH("scatter_rows");
  return ALODLM_OK;
}

extern "C" int alodlm_cross_entropy(void* logits, const int32_t* target, const float* coef,
                                    const int32_t* n_rows, int64_t max_rows, int64_t vocab,
                                    float* ce, float* entropy, int dtype, void* stream) {
  ALODLM_CHECK_ARG(vocab > 0, "cross_entropy: bad vocab");
  if (max_rows == 0) return ALODLM_OK;
  const bool v8 = vocab % 8 == 0 && aligned8(logits, dtype);
  if (v8 && dtype == ALODLM_BF16 && vocab > 8 * CE_THREADS * (CE_ROW_NCH / 2) &&
      vocab <= 8 * CE_THREADS * CE_ROW_NCH) {
    // one workgroup per CU (its threads hold a whole row), each walking rows
    const int64_t cus = device_cus();
    const int64_t grid = max_rows < cus ? max_rows : cus;
    cross_entropy_row_kernel<CE_ROW_NCH><<<(unsigned)grid, CE_THREADS, 0, as_stream(stream)>>>(
        (bf16_t*)logits, target, coef, n_rows, vocab, ce, entropy);
    ALODLM_CHECK_LAUNCH("cross_entropy_row");
    return ALODLM_OK;
  }
  ALODLM_DISPATCH(dtype, T, {
    if (v8) cross_entropy_kernel<T, true><<<(unsigned)max_rows, 256, 0, as_stream(stream)>>>(
        (T*)logits, target, coef, n_rows, vocab, ce, entropy);
    else cross_entropy_kernel<T, false><<<(unsigned)max_rows, 256, 0, as_stream(stream)>>>(
        (T*)logits, target, coef, n_rows, vocab, ce, entropy);
  });
  ALODLM_CHECK_LAUNCH("cross_entropy");
  return ALODLM_OK;
}

// Decode readout (alodlm/inference.py:115-118): per row of logits, the index
// of the largest logit (the first one among equal maxima, like torch.argmax)
// and the entropy -sum p log p = lse - sum p * x of the softmax, in float32.
// The logits are left unchanged.  One 256-thread block per row.
template <typename T>
__global__ void __launch_bounds__(256)
decode_readout_kernel(const T* __restrict__ logits, int64_t V, int64_t* __restrict__ argmax,
                      float* __restrict__ entropy) {
  __shared__ float sm[4], ss[4], st[4], bv[4];
  __shared__ int64_t bi[4];
  const T* lr = logits + (int64_t)blockIdx.x * V;
  float m = -INFINITY, s = 0.f, t = 0.f, best = -INFINITY;
  int64_t best_i = V;
  for (int64_t c = threadIdx.x; c < V; c += 256) {
    const float x = Elem<T>::load(lr, c);
    if (x > best) { best = x; best_i = c; }  // a thread's indices increase
    if (x > m) {
      const float scale = expf(m - x);
      s = s * scale + 1.f;
      t = t * scale + x;
      m = x;
    } else {
      const float e = expf(x - m);
      s += e;
      t += e * x;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // argmax across the wavefront: larger value, or equal value and smaller index
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int64_t oi = __shfl_xor(best_i, off, 64);
    if (ov > best || (ov == best && oi < best_i)) { best = ov; best_i = oi; }
  }
  const float M = wave_max(m);
  const float scale = (m == -INFINITY) ? 0.f : expf(m - M);
  const float S = wave_sum(s * scale), Tt = wave_sum(t * scale);
  if (lane == 0) { sm[wave] = M; ss[wave] = S; st[wave] = Tt; bv[wave] = best; bi[wave] = best_i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float gm = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
    float gs = 0.f, gt = 0.f, gv = bv[0];
    int64_t gi = bi[0];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = (sm[w] == -INFINITY) ? 0.f : expf(sm[w] - gm);
      gs += ss[w] * f;
      gt += st[w] * f;
      if (bv[w] > gv || (bv[w] == gv && bi[w] < gi)) { gv = bv[w]; gi = bi[w]; }
    }
    argmax[blockIdx.x] = gi;
    entropy[blockIdx.x] = gm + logf(gs) - gt / gs;
  }
}

extern "C" int alodlm_decode_readout(const void* logits, int64_t rows, int64_t vocab,
                                     int64_t* argmax, float* entropy, int dtype, void* stream) {
  ALODLM_CHECK_ARG(rows >= 0 && vocab > 0, "decode_readout: bad shape");
  ALODLM_CHECK_ARG(rows <= 0x7fffffff, "decode_readout: too many rows");
  if (rows == 0) return ALODLM_OK;
  ALODLM_DISPATCH(dtype, T, {
    decode_readout_kernel<T><<<(unsigned)rows, 256, 0, as_stream(stream)>>>(
        (const T*)logits, vocab, argmax, entropy);
  });
  ALODLM_CHECK_LAUNCH("decode_readout");
  return ALODLM_OK;
}

extern "C" int alodlm_scatter_ce(const float* ce, const int32_t* sel_rows, const int32_t* n_rows,
                                 int64_t max_rows, float* ce_full, int64_t rows, void* stream) {
  (void)rows;
  if (max_rows == 0) return ALODLM_OK;
  scatter_ce_kernel<<<ceil_div_u(max_rows, 256), 256, 0, as_stream(stream)>>>(ce, sel_rows, n_rows,
                                                                             max_rows, ce_full);
  ALODLM_CHECK_LAUNCH("scatter_ce");
  return ALODLM_OK;
}

extern "C" int64_t alodlm_gate_bwd_workspace(int64_t rows, int64_t hidden) {
  return ((rows + kGateBwdRows - 1) / kGateBwdRows) * (hidden + 1);
}

extern "C" int alodlm_gate_bwd(const float* dgate, const void* readout, float scale,
                               float* gw_accum, float* gb_accum, float* gdb_accum, int64_t depth,
                               int64_t rows, int64_t hidden, float* workspace, int dtype,
                               void* stream) {
  ALODLM_CHECK_ARG(rows > 0 && hidden > 0, "gate_bwd: bad shape");
  const int64_t nparts = (rows + kGateBwdRows - 1) / kGateBwdRows;
  ALODLM_CHECK_ARG(nparts <= 65535, "gate_bwd: too many rows");
  hipStream_t st = as_stream(stream);
  const bool v8 = hidden % 8 == 0 && aligned8(readout, dtype);
  ALODLM_DISPATCH(dtype, T, {
    if (v8)
      gate_bwd_kernel<T, true><<<dim3(ceil_div_u(hidden, 8 * 256), (unsigned)nparts), 256, 0, st>>>(
          dgate, (const T*)readout, workspace, rows, hidden, kGateBwdRows);
    else
      gate_bwd_kernel<T, false><<<dim3(ceil_div_u(hidden, 256), (unsigned)nparts), 256, 0, st>>>(
          dgate, (const T*)readout, workspace, rows, hidden, kGateBwdRows);
  });
  ALODLM_CHECK_LAUNCH("gate_bwd");
  gate_bwd_reduce_kernel<<<ceil_div_u(hidden + 1, 256), 256, 0, st>>>(
      workspace, nparts, hidden, scale, gw_accum, gb_accum, gdb_accum + depth);
  ALODLM_CHECK_LAUNCH("gate_bwd_reduce");
  return ALODLM_OK;
}
