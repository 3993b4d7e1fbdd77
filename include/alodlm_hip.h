/*
 * alodlm_hip.h - C ABI of the MI355X (gfx950) kernels behind the ALoDLM
 * training step.
 *
 * Conventions
 *   - Every entry point is stateless, enqueues work on `stream` (a hipStream_t
 *     passed as void*; NULL = the default stream) and returns ALODLM_OK or an
 *     error code; alodlm_last_error() then holds a message.  Nothing
 *     synchronises the device unless stated.
 *   - Pointers are device pointers unless named host_*.  The caller owns all
 *     memory: outputs and workspaces are allocated by the caller.
 *   - `dtype` selects the storage type of activations and weights:
 *     ALODLM_F32 (float) or ALODLM_BF16 (bfloat16, 2 bytes).  Arithmetic is
 *     float32; bf16 results are rounded to nearest even at the same points
 *     where the reference's bf16 eager ops round.
 *   - Row-major matrices; `ld*` are row strides in elements.
 *
 * Citations name the reference function each entry point replaces
 * (amazon-science/ALoDLM; [tf] = transformers' Qwen3 modules).
 */
#ifndef ALODLM_HIP_H
#define ALODLM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ALODLM_ABI_VERSION 7

enum { ALODLM_OK = 0, ALODLM_EINVAL = 1, ALODLM_EHIP = 2, ALODLM_EUNSUPPORTED = 3 };
enum { ALODLM_F32 = 0, ALODLM_BF16 = 1 };

/* Library identity and errors. */
int alodlm_abi_version(void);
const char* alodlm_last_error(void);
/* Compute units and peak engine clock (kHz) of a device, for the peak
 * figures measurements are quoted against.  No counterpart in the reference
 * (its benchmarks read them from the vendor tools). */
int alodlm_device_info(int device, int64_t* compute_units, int64_t* max_clock_khz);

/* ---------------------------------------------------------------------------
 * Masking draws (alodlm/batch.py:50-60): the values of the reference's
 * per-segment `uniform_(0, 1).clamp_min(1e-8)` and per-masked-block
 * `randperm(n_cand)` calls on a Philox device generator whose state on entry
 * is (seed, offset), evaluated in two launches.  block_n[b] is block b's
 * candidate count (labels != -100, 0..block_size); segment s owns blocks
 * [seg_block[s], seg_block[s+1]).  key_bits[n] (n = 0..block_size) is the
 * randperm sort-key width.  Writes block_p, block_count = round(n * p),
 * block_offset (the generator offset of each block's randperm), perm_offset
 * = b * block_size, perms (n_blocks * block_size int64; block b's randperm
 * at perm_offset[b] when block_count[b] > 0) and *offset_out, the generator
 * offset after every draw.  Replaces the per-block torch calls of
 * alodlm/batch.py:50-60; the output feeds alodlm_batch_build.
 * ------------------------------------------------------------------------ */
int alodlm_mask_draws(uint64_t seed, uint64_t offset, const int32_t* seg_block,
                      int64_t n_segments, const int32_t* block_n, int64_t n_blocks,
                      int64_t block_size, const int32_t* key_bits, float* block_p,
                      int32_t* block_count, uint64_t* block_offset, int64_t* perm_offset,
                      int64_t* perms, uint64_t* offset_out, void* stream);

/* ---------------------------------------------------------------------------
 * Dual-stream batch (alodlm/batch.py:34-85, build_batch).
 * Given the masking draws (per-block mask probability `block_p`,
 * per-block masked count `block_count` = round(n_candidates * p) and the
 * concatenated randperm draws `perms` with per-block offsets `perm_offset`),
 * writes the clean+noisy rows of every segment.  Segment s covers tokens
 * [seg[s], seg[s+1]) and dual-stream rows [2*seg[s], 2*seg[s+1]); its blocks
 * are [seg_block[s], seg_block[s+1]).  Outputs have 2*n_tokens rows:
 * out_ids / out_original / out_positions (int64), out_masked (uint8),
 * out_prob (float), row_segment (int32), ar_target (int32: the next-token
 * label of a clean row or -1, alodlm/loss.py:20-25) and out_boundaries
 * (int64, S+1).
 * ------------------------------------------------------------------------ */
int alodlm_batch_build(const int64_t* ids, const int64_t* labels, const int64_t* seg,
                       const int32_t* seg_block, int64_t n_segments, int64_t n_blocks,
                       int64_t block_size, int64_t mask_token_id, const float* block_p,
                       const int32_t* block_count, const int64_t* perm_offset,
                       const int64_t* perms, int64_t* out_ids, int64_t* out_original,
                       int64_t* out_positions, uint8_t* out_masked, float* out_prob,
                       int32_t* row_segment, int32_t* ar_target, int64_t* out_boundaries,
                       void* stream);

/* ---------------------------------------------------------------------------
 * Embedding ([tf] modeling_qwen3.py:352; alodlm/model.py:133,149).
 * gather: out[r] = table[ids[r]].  Ids outside [0, vocab) give NaN rows
 * (gather) or no gradient (scatter); they are never dereferenced.
 *
 * The backward is deterministic: embed_plan sorts the rows by id (stable,
 * one workgroup) into runs of equal ids cut into chunks of at most 32 rows;
 * plan holds alodlm_embed_plan_size(rows) int32 and serves every later
 * scatter over the same ids (rows < 2^24).  scatter_add: dtable[ids[r]] +=
 * dout[r] (float32) for rows with row_exits == NULL or row_exits[r] <=
 * max_exit, each chunk summed in row order and the chunks of a run in chunk
 * order, so the result does not depend on scheduling (the reference's
 * nn.Embedding backward accumulates with atomics).  workspace holds
 * alodlm_embed_scatter_workspace(rows, hidden) floats.
 * ------------------------------------------------------------------------ */
int alodlm_embed_gather(const void* table, const int64_t* ids, void* out, int64_t rows,
                        int64_t hidden, int64_t vocab, int dtype, void* stream);
int64_t alodlm_embed_plan_size(int64_t rows);
int alodlm_embed_plan(const int64_t* ids, int64_t rows, int64_t vocab, int32_t* plan,
                      void* stream);
int64_t alodlm_embed_scatter_workspace(int64_t rows, int64_t hidden);
int alodlm_embed_scatter_add(const void* dout, const int32_t* plan, const int32_t* row_exits,
                             int64_t max_exit, float* dtable, float* workspace, int64_t rows,
                             int64_t hidden, int64_t vocab, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * RMSNorm ([tf] modeling_qwen3.py:59-64): y = w * cast(x * rsqrt(mean(x^2) + eps)).
 * fwd writes y and rstd[rows] (float).
 * bwd: dx = dres + d(norm)/dx . dy (dres may be NULL; dx may alias dres);
 * dw_accum[cols] += sum_rows dy * cast(x*rstd) using `workspace` of
 * alodlm_rmsnorm_bwd_workspace(rows, cols) floats (deterministic order).
 * ------------------------------------------------------------------------ */
int alodlm_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows,
                       int64_t cols, float eps, int dtype, void* stream);
int64_t alodlm_rmsnorm_bwd_workspace(int64_t rows, int64_t cols);
int alodlm_rmsnorm_bwd(const void* dy, const void* x, const float* rstd, const void* w,
                       const void* dres, void* dx, float* dw_accum, float* workspace,
                       int64_t rows, int64_t cols, int dtype, void* stream);

/* alodlm_rmsnorm_bwd without a workspace argument and without any device
 * allocation.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Its scratch is a library-held device
 * array of ALODLM_NOALLOC_SCRATCH_FLOATS floats per GPU (16 MiB, held until
 * the process ends); shapes whose alodlm_rmsnorm_bwd_workspace(rows, cols)
 * exceeds it return ALODLM_EINVAL (e.g. 32768 x 2048 and 4096 x 4096 fit,
 * 65536 x 2048 does not).  Results are bit-identical to alodlm_rmsnorm_bwd.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (different streams or threads without ordering) race; calls ordered on
 * one stream are safe. */
#define ALODLM_NOALLOC_SCRATCH_FLOATS 4194304
int alodlm_rmsnorm_bwd_noalloc(const void* dy, const void* x, const float* rstd, const void* w,
                               const void* dres, void* dx, float* dw_accum, int64_t rows,
                               int64_t cols, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * q_norm/k_norm + rotary (alodlm/model.py:41-46,58; [tf] :126-137).
 * qkv: [rows, (nq+2*nkv)*dh] projections (q | k | v).  positions: int64 [rows].
 * inv_freq: float [dh/2].  fwd writes q_out [rows, nq*dh] and k_out
 * [rows, nkv*dh] (normalised, rotated).  bwd takes dq, dk of the rotated
 * values, recomputes the forward, writes dqkv's q and k columns and adds the
 * norm-weight gradients into dwq_accum/dwk_accum (float, dh each) using
 * `workspace` of alodlm_qknorm_rope_bwd_workspace(rows, nq, nkv, dh) floats.
 * ------------------------------------------------------------------------ */
int alodlm_qknorm_rope_fwd(const void* qkv, const void* wq, const void* wk,
                           const int64_t* positions, const float* inv_freq, void* q_out,
                           void* k_out, int64_t rows, int64_t nq, int64_t nkv, int64_t dh,
                           float eps, int dtype, void* stream);
int64_t alodlm_qknorm_rope_bwd_workspace(int64_t rows, int64_t nq, int64_t nkv, int64_t dh);
int alodlm_qknorm_rope_bwd(const void* dq, const void* dk, const void* qkv, const void* wq,
                           const void* wk, const int64_t* positions, const float* inv_freq,
                           void* dqkv, float* dwq_accum, float* dwk_accum, float* workspace,
                           int64_t rows, int64_t nq, int64_t nkv, int64_t dh, float eps,
                           int dtype, void* stream);
/* The same with the rotation read from caller tables cos_tab / sin_tab
 * [rows, dh] in the storage dtype (the cos, sin arguments of
 * alodlm/model.py:41-46 and layer_forward, model.py:49-58), element i of
 * each head rotating with entry i of its row. */
int alodlm_qknorm_rotary_fwd(const void* qkv, const void* wq, const void* wk, const void* cos_tab,
                             const void* sin_tab, void* q_out, void* k_out, int64_t rows,
                             int64_t nq, int64_t nkv, int64_t dh, float eps, int dtype,
                             void* stream);
int alodlm_qknorm_rotary_bwd(const void* dq, const void* dk, const void* qkv, const void* wq,
                             const void* wk, const void* cos_tab, const void* sin_tab, void* dqkv,
                             float* dwq_accum, float* dwk_accum, float* workspace, int64_t rows,
                             int64_t nq, int64_t nkv, int64_t dh, float eps, int dtype,
                             void* stream);
/* The rotary alone (alodlm/model.py:41-46, `rotary`): out = x * cos +
 * rotate_half(x) * sin for x [rows, heads, dh] and tables [rows, dh], each
 * product and the sum rounded to the storage dtype; bwd gives dx from dout
 * (the transposed rotation, rounded like the reference's bf16 autograd). */
int alodlm_rotary_fwd(const void* x, const void* cos_tab, const void* sin_tab, void* out,
                      int64_t rows, int64_t heads, int64_t dh, int dtype, void* stream);
int alodlm_rotary_bwd(const void* dout, const void* cos_tab, const void* sin_tab, void* dx,
                      int64_t rows, int64_t heads, int64_t dh, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * GEMM for every linear layer (nn.Linear at alodlm/model.py:55-57,74-75,161;
 * [tf] :81-83, replaced cuBLAS calls).
 *   C[m, n] = alpha * sum_k A(m, k) * B(n, k)      (float32 accumulation)
 * a_kmajor != 0: A(m,k) = A[m*lda + k]  (row-major [M,K]);
 *          == 0: A(m,k) = A[k*lda + m]  (row-major [K,M]).
 * b_kmajor != 0: B(n,k) = B[n*ldb + k]  (row-major [N,K], i.e. nn.Linear's W);
 *          == 0: B(n,k) = B[k*ldb + n]  (row-major [K,N]).
 * epilogue: ALODLM_EPI_STORE    C = alpha*acc                (C in dtype)
 *           ALODLM_EPI_RESIDUAL C = R + cast(alpha*acc)       (C, R in dtype; may alias)
 *           ALODLM_EPI_ACCUM    Cf32 += alpha*acc             (C is float)
 *           ALODLM_EPI_STORE_F32 Cf32 = alpha*acc            (C is float: the first
 *                               contribution to a gradient, which then needs no zeroing)
 * workspace: float scratch of alodlm_gemm_workspace(M, N, K, epilogue, dtype)
 * floats for split-K partials: ALODLM_EPI_ACCUM products with few output
 * tiles, and bf16 ALODLM_EPI_STORE products with K >= 16384 and few output
 * tiles (summed in split order, then rounded once).  May be NULL (the
 * product then runs unsplit); unused when the query returns 0.
 * ------------------------------------------------------------------------ */
enum { ALODLM_EPI_STORE = 0, ALODLM_EPI_RESIDUAL = 1, ALODLM_EPI_ACCUM = 2,
       ALODLM_EPI_STORE_F32 = 3 };
int64_t alodlm_gemm_workspace(int64_t M, int64_t N, int64_t K, int epilogue, int dtype);
int alodlm_gemm(const void* A, int64_t lda, int a_kmajor, const void* B, int64_t ldb,
                int b_kmajor, void* C, int64_t ldc, const void* R, int64_t ldr, int64_t M,
                int64_t N, int64_t K, float alpha, int epilogue, int dtype, float* workspace,
                void* stream);
/* The weight gradient of a layer applied once per recurrent pass
 * (alodlm/model.py:152, the loop over depths, whose autograd sums the passes'
 * nn.Linear weight gradients) as one product:
 *   C[m, n] (=|+=) alpha * sum_i sum_k A_i[k*lda + m] * B_i[k*ldb + n]
 * over nseg (1..8) segments of seg_k k rows each (a multiple of 32), A_i =
 * a_segs[i], B_i = b_segs[i] (bf16, m/n-contiguous like alodlm_gemm with
 * a_kmajor = b_kmajor = 0, 16-byte aligned), C float32; epilogue
 * ALODLM_EPI_STORE_F32 or ALODLM_EPI_ACCUM.  M, N >= 256 and multiples of 8.
 * workspace: alodlm_gemm_workspace(M, N, nseg * seg_k, epilogue, bf16)
 * floats, or NULL.  One float32 sum runs through the segments in order. */
int alodlm_gemm_segk(const void* const* a_segs, const void* const* b_segs, int nseg,
                     int64_t seg_k, int64_t lda, int64_t ldb, void* C, int64_t ldc, int64_t M,
                     int64_t N, float alpha, int epilogue, float* workspace, void* stream);

/* ---------------------------------------------------------------------------
 * GQA attention under the dual-stream training mask (alodlm/model.py:62-73
 * with the mask of alodlm/batch.py:23-31, or equivalently the range plan of
 * alodlm/attention.py:12-30).  q: [rows, nq*dh]; k: [rows, nkv*dh];
 * v: rows of stride ldv; o: [rows, nq*dh]; lse: float [nq, rows].
 * Segment s spans dual-stream rows [bounds[s], bounds[s+1]) (clean half
 * first); row_segment[r] = s.  Scale is dh^-0.5.
 * tiles: int32 [n_tiles, 2] = (segment, in-segment start row) of every
 * 128-row tile of every stream (a tile never crosses a stream); with tiles,
 * bf16 and head_dim 64/128 the MFMA flash kernels run, otherwise (or with
 * tiles == NULL) the reference kernels.
 * bwd: dq [rows, nq*dh], dk [rows, nkv*dh], dv (stride lddv) from do.
 * `workspace` holds alodlm_attention_bwd_workspace(rows, nq, nkv, dh, n_tiles,
 * ds_blocks) floats (delta per head and row; for head_dim 128 also
 * lse * log2(e) per head and row, the dK/dV pass's work counter, with few key
 * tiles per kv head float32 dK/dV partials per query head, and the stored dS
 * blocks).  Calls that share a workspace must not overlap.
 * Stored dS (head_dim 128, bf16, block_size 32): with ds_base (device int64
 * [S+1], each segment's first 32x32 block as alodlm_attention_ds_blocks
 * fills it) and ds_blocks (its total, > 0), the dK/dV pass stores the bf16 dS
 * of every allowed pair and dQ is one dS*K product over them, instead of
 * recomputing S, P and dP; ds_base NULL (or ds_blocks 0, or a buffer of
 * nq * ds_blocks * 2 KiB at or above 2 GiB) selects the recomputing dQ pass.
 * alodlm_attention_ds_blocks is host code: token_offsets are the S+1 token
 * offsets of the pack (host memory).
 * ------------------------------------------------------------------------ */
int alodlm_attention_fwd(const void* q, const void* k, const void* v, int64_t ldv,
                         const int64_t* bounds, const int32_t* row_segment,
                         const int32_t* tiles, int64_t n_tiles, void* o, float* lse,
                         int64_t rows, int64_t nq, int64_t nkv, int64_t dh, int64_t block_size,
                         int dtype, void* stream);
int64_t alodlm_attention_ds_blocks(const int64_t* token_offsets, int64_t segments,
                                   int64_t block_size, int64_t* base_out);
int64_t alodlm_attention_bwd_workspace(int64_t rows, int64_t nq, int64_t nkv, int64_t dh,
                                       int64_t n_tiles, int64_t ds_blocks);
int alodlm_attention_bwd(const void* q, const void* k, const void* v, int64_t ldv,
                         const void* o, const float* lse, const void* dout,
                         const int64_t* bounds, const int32_t* row_segment,
                         const int32_t* tiles, int64_t n_tiles, void* dq, void* dk, void* dv,
                         int64_t lddv, float* workspace, const int64_t* ds_base,
                         int64_t ds_blocks, int64_t rows, int64_t nq, int64_t nkv, int64_t dh,
                         int64_t block_size, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * SwiGLU ([tf] modeling_qwen3.py:81-83): gu = [gate | up] of width 2*inter;
 * fwd act = cast(cast(silu(gate)) * up); bwd dgu from dact.
 * ------------------------------------------------------------------------ */
int alodlm_swiglu_fwd(const void* gu, void* act, int64_t rows, int64_t inter, int dtype,
                      void* stream);
/* act (nullable): also write the forward product, bit-identical to
 * alodlm_swiglu_fwd's, so the backward needs no separate recompute pass. */
int alodlm_swiglu_bwd(const void* dact, const void* gu, void* dgu, void* act, int64_t rows,
                      int64_t inter, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Readout and halting (alodlm/model.py:152-168).
 * final_norm_gate: readout = norm(x) (the model's final RMSNorm, weight wf)
 *   and gate[r] = (readout . gate_w + gate_b) + depth_bias[depth]
 *   (GateHead.forward, model.py:37-38), rounded like the reference; gate is
 *   stored as float.  rstd: float [rows].
 * carry_select: at depth d >= 1, out[r] = table[original[r]] if exits[r] <= d
 *   (re-embedding, model.py:153-154) else norm(x)[r] (the carry, model.py:168);
 *   writes rstd of the carry norm.
 * exit_update (model.py:163-167): for d < K-1, exits[r] = d+1 where
 *   u[r] < sigmoid(gate[r]) and masked[r] and exits[r] == K.
 * ------------------------------------------------------------------------ */
int alodlm_final_norm_gate(const void* x, const void* wf, const void* gate_w,
                           const void* gate_b, const void* depth_bias, int64_t depth,
                           void* readout, float* rstd, float* gate, int64_t rows,
                           int64_t hidden, float eps, int dtype, void* stream);
int alodlm_carry_select(const void* x, const void* wf, const void* table,
                        const int64_t* original, const int32_t* exits, int64_t depth,
                        void* out, float* rstd, int64_t rows, int64_t hidden, int64_t vocab,
                        float eps, int dtype, void* stream);
/* Backward of carry_select at depth d: rows with exits <= d add dy into
 * dtable[original] (float; plan = alodlm_embed_plan of original); the others
 * go through the carry norm: dx = dres + norm'(x) . dy, dwf_accum += ...;
 * re-embedded rows get dx = dres.  workspace holds
 * alodlm_carry_select_bwd_workspace(rows, hidden) floats. */
int64_t alodlm_carry_select_bwd_workspace(int64_t rows, int64_t hidden);
int alodlm_carry_select_bwd(const void* dy, const void* x, const float* rstd, const void* wf,
                            const int32_t* exits, int64_t depth, const int32_t* plan,
                            const void* dres, void* dx, float* dwf_accum, float* dtable,
                            float* workspace, int64_t rows, int64_t hidden, int64_t vocab,
                            int dtype, void* stream);
int alodlm_exit_update(const float* gate, const float* uniforms, const uint8_t* masked,
                       int32_t* exits, int64_t depth, int64_t max_depth, int64_t rows,
                       void* stream);

/* ---------------------------------------------------------------------------
 * Readout row selection for depth d (model.py:180-184; loss.py:12-32):
 * a row carries loss at depth d if it is masked and not yet exited before d
 * (target original[r], coefficient dL/dce = 0.5 * w_r * stick[d, r], from
 * loss.py:55-61) or it is a clean row with an autoregressive target
 * (target ar_target[r] >= 0, coefficient ar_coef).  Writes the selected row
 * indices in ascending order, their targets and coefficients, and the count
 * (device int32).  gates: float [K, rows]; wsum: device float holding
 * sum over masked rows of 1/(p+1e-8).
 * ------------------------------------------------------------------------ */
int alodlm_select_rows(const uint8_t* masked, const int32_t* exits, const int64_t* original,
                       const int32_t* ar_target, const float* gates, const float* mask_prob,
                       const float* wsum, float ar_coef, int64_t depth, int64_t max_depth,
                       int64_t rows, int32_t* sel_rows, int32_t* sel_target, float* sel_coef,
                       int32_t* sel_count, void* stream);
int alodlm_inverse_weight_sum(const uint8_t* masked, const float* mask_prob, int64_t rows,
                              float* wsum, void* stream);

/* Row gather/scatter between the full [rows, H] stream and the selected rows. */
int alodlm_gather_rows(const void* src, const int32_t* sel_rows, int64_t n_sel, void* dst,
                       int64_t hidden, int dtype, void* stream);
int alodlm_scatter_rows(const void* src, const int32_t* sel_rows, int64_t n_sel, void* dst,
                        int64_t rows, int64_t hidden, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Cross-entropy over the vocabulary for the selected rows (F.cross_entropy
 * at model.py:180 and loss.py:24-25), fused with token entropy:
 * logits [n, V] (dtype) -> ce[n] = lse - logit[target] (rounded to dtype like
 * the reference's CE output), entropy[n] = lse - sum p*logit, and in place
 * logits <- coef * (softmax - onehot(target)), i.e. dL/dlogits per unit of
 * upstream gradient.  Rows beyond n_rows (device count) are untouched.
 * ------------------------------------------------------------------------ */
int alodlm_cross_entropy(void* logits, const int32_t* target, const float* coef,
                         const int32_t* n_rows, int64_t max_rows, int64_t vocab, float* ce,
                         float* entropy, int dtype, void* stream);
/* Decode readout (alodlm/inference.py:115-118: logits.argmax(-1) and the
 * entropy -(exp(logp) * logp).sum(-1) of log_softmax(logits.float())):
 * logits [rows, V] (dtype, unchanged) -> argmax[rows] (int64; the first index
 * among equal maxima) and entropy[rows] (float). */
int alodlm_decode_readout(const void* logits, int64_t rows, int64_t vocab, int64_t* argmax,
                          float* entropy, int dtype, void* stream);
/* ---------------------------------------------------------------------------
 * Adaptive decoding's window bookkeeping (alodlm/inference.py:71-246) on the
 * device.  The state is a set of caller-allocated device arrays:
 *   ledger   the pending tail of the text in logical order (capacity slots):
 *            slot_token, slot_open (1 = still a mask token), slot_depth and
 *            slot_halt (exit depth and first-pass halt probability of a
 *            committed slot);
 *   output   out_token / out_depth / out_halt (max_new_tokens entries);
 *   window   row_token / row_position (window rows: committed slots, then
 *            open slots, each in logical order; position = cache rows +
 *            slot), and per mask row j: mask_row (window row), mask_slot,
 *            mask_offset (position penalty: (slot_j - slot_0) * penalty),
 *            mask_token / mask_exit / mask_committed / mask_fresh (committed
 *            at the current depth), mask_survival, mask_first_hazard;
 *   readout  predicted / entropy of the mask rows at the current depth
 *            (alodlm_decode_readout writes them);
 *   carry    replace_token / replace_depth of the window rows: the next
 *            depth's alodlm_carry_select table (rows committed at depth d
 *            restart from their token's embedding at depth d + 1);
 *   header   ALODLM_DECODE_HEADER int64 fields, indices below.
 * One workgroup per call; the caller reads the header after a commit.
 * ------------------------------------------------------------------------ */
#define ALODLM_DECODE_HEADER 16
enum {
  ALODLM_DECODE_LEDGER = 0,     /* ledger slots in use */
  ALODLM_DECODE_GENERATED = 1,  /* tokens in the output stream */
  ALODLM_DECODE_CACHE = 2,      /* cached prefix rows (retired tokens + prompt) */
  ALODLM_DECODE_DONE = 3,       /* 1 once decoding has ended */
  ALODLM_DECODE_REASON = 4,     /* ALODLM_DECODE_LENGTH or ALODLM_DECODE_EOS */
  ALODLM_DECODE_WINDOW = 5,     /* rows of the planned window */
  ALODLM_DECODE_OBSERVED = 6,   /* committed rows at its start (mask rows follow) */
  ALODLM_DECODE_PREFIX = 7,     /* leading committed slots it retires when it ends */
  ALODLM_DECODE_STOP = 8        /* 1 when the last committed depth ended the window */
};
enum { ALODLM_DECODE_LENGTH = 0, ALODLM_DECODE_EOS = 1 };
enum { ALODLM_DECODE_ENTROPY = 0, ALODLM_DECODE_LEFT1 = 1 };
typedef struct {
  int64_t* slot_token; int32_t* slot_open; int32_t* slot_depth; float* slot_halt;
  int64_t* out_token; int32_t* out_depth; float* out_halt;
  int64_t* row_token; int64_t* row_position;
  int32_t* mask_row; int32_t* mask_slot; float* mask_offset;
  int64_t* mask_token; int32_t* mask_exit; int32_t* mask_committed; int32_t* mask_fresh;
  float* mask_survival; float* mask_first_hazard;
  int64_t* predicted; float* entropy;
  int64_t* replace_token; int32_t* replace_depth;
  int64_t* header;
  const int64_t* stop_ids; int64_t n_stop;
  int64_t capacity;        /* rows of the window and mask arrays, slots of the ledger */
  int64_t max_new_tokens, window_size, mask_token_id, max_depth;
  float tau, q, penalty;   /* DecodeConfig.tau, .q and the position penalty */
  int32_t mode;            /* ALODLM_DECODE_ENTROPY or ALODLM_DECODE_LEFT1 */
} alodlm_decode_state;
/* The top of the decoding loop (inference.py:185-210) from the header's
 * ledger, output and cache counts: ends decoding (emitting the committed
 * run up to a stop token) or grows the ledger to the window size and lays
 * out the window.  capacity >= 2 * window_size. */
int alodlm_decode_plan(const alodlm_decode_state* state, void* stream);
/* Fresh mask-row state for a window given by the caller (rows rows, the
 * count mask rows at logical positions logical[count]); replace_depth of
 * every row = max_depth.  alodlm_decode_plan does this itself. */
int alodlm_decode_begin(const alodlm_decode_state* state, const int64_t* logical, int64_t rows,
                        int64_t count, void* stream);
/* One depth's commitments (inference.py:109-142): hazard = sigmoid(gate[row])
 * of each mask row, survival, the entropy (tau) or left-to-right agreement,
 * the stop rule (last depth, nothing left, or mean (1 - survival) of the
 * uncommitted rows >= q) and its fallback (least adjusted entropy commits),
 * and the next depth's carry table; header[STOP] says whether the window
 * ended.  With `finish`, an ended window is retired (inference.py:227-238:
 * the committed run it started with is emitted and stays cached, its
 * commitments go to their slots) and the next one planned. */
int alodlm_decode_commit(const alodlm_decode_state* state, const float* gate, int64_t count,
                         int64_t depth, int finish, void* stream);

/* Scatter ce of the selected rows into ce_full[depth, rows]. */
int alodlm_scatter_ce(const float* ce, const int32_t* sel_rows, const int32_t* n_rows,
                      int64_t max_rows, float* ce_full, int64_t rows, void* stream);

/* ---------------------------------------------------------------------------
 * Objective (alodlm/loss.py:35-90, alodlm/credit.py:7-40, model.py:183-187).
 * Inputs over all rows: gates [K, rows], exits, masked, mask_prob,
 * ce_full [K, rows] (valid where masked and d < z), ar_ce [K, rows]
 * (valid where ar_target >= 0), row_segment, bounds [S+1].
 * out[0..9] = total, denoising, actor, sampled_mean_depth, prediction_cost,
 *   regularization_cost, profile_mean_depth, first_pass_halt_probability,
 *   ar_loss, masked_count.
 * dgate [K, rows] = d total / d gate (unit upstream gradient).
 * total is NaN when a gate is non-finite or when `nonfinite` (nullable) holds
 * a nonzero value: the reference adds 0 * sum(logits + gates) to the loss
 * (model.py:186), and the step sets that flag when an LM-head weight is
 * non-finite (alodlm_check_finite), which makes a logits column
 * non-finite in every row, computed or not.
 * One workgroup; `workspace` holds alodlm_objective_workspace(rows, S, K) floats.
 * ------------------------------------------------------------------------ */
int64_t alodlm_objective_workspace(int64_t rows, int64_t n_segments, int64_t max_depth);
int alodlm_objective(const float* gates, const int32_t* exits, const uint8_t* masked,
                     const float* mask_prob, const float* ce_full, const float* ar_ce,
                     const int32_t* ar_target, const int64_t* bounds, int64_t n_segments,
                     int64_t rows, int64_t max_depth, float depth_prior_c, float kl_beta_mi,
                     float kl_beta_marg, const int32_t* nonfinite, float* out, float* dgate,
                     float* workspace, void* stream);
/* outcome_loss alone (alodlm/loss.py:35-90): the objective above without the
 * autoregressive part; out[0..9] as above with out[0] = (denoising + actor)
 * / 2 and out[8] = 0, so the outcome loss is out[1] + out[2].  dgate [K, rows]
 * = d(denoising + actor)/d gate and dce [K, rows] = d(denoising)/d ce (the
 * row's weight times the detached stick at d < z, else 0).  Same workspace as
 * alodlm_objective. */
int alodlm_outcome_loss(const float* gates, const int32_t* exits, const uint8_t* masked,
                        const float* mask_prob, const float* ce_full, const int64_t* bounds,
                        int64_t n_segments, int64_t rows, int64_t max_depth, float depth_prior_c,
                        float kl_beta_mi, float kl_beta_marg, float* out, float* dgate,
                        float* dce, float* workspace, void* stream);
/* masked_sequence_ids (alodlm/credit.py:7-21): out[j] = segment of the j-th
 * masked row in row order (bucketize(rows, bounds[1:], right=True)[masked]),
 * *count = number of masked rows (device int64).  bounds [S+1] as the
 * caller's cum_seqlens; the host-side validation of credit.py:8-19 stays with
 * the caller.  One workgroup. */
int alodlm_masked_sequence_ids(const uint8_t* masked, const int64_t* bounds, int64_t n_segments,
                               int64_t rows, int64_t* out, int64_t* count, void* stream);
/* sequence_score_function (alodlm/credit.py:23-40): value[0] =
 * sum_s R_s Q_s / n with R_s, Q_s the per-sequence sums of credit and logq
 * (rows in order within a sequence), dlogq[i] = R_{ids[i]} / n.  ids in
 * [0, sequence_count); `workspace` holds 2 * sequence_count floats.  One
 * workgroup, one wavefront per sequence (cost n * sequence_count / 1024). */
int alodlm_sequence_score(const float* credit, const float* logq, const int64_t* ids, int64_t n,
                          int64_t sequence_count, float* value, float* dlogq, float* workspace,
                          void* stream);
/* Next-token targets of autoregressive_loss (alodlm/loss.py:12-32) over the
 * dual-stream rows: clean row start + i of a segment [start, end) with
 * L = (end - start) / 2 >= 2 and i < L - 1 predicts labels[start/2 + 1 + i];
 * every other row and ignored labels (-100) get -1. */
int alodlm_ar_targets(const int64_t* labels, const int64_t* bounds, int64_t n_segments,
                      int64_t rows, int32_t* target, void* stream);

/* Gate-head backward (GateHead.forward, model.py:37-38, differentiated):
 * gw_accum[H] += scale * sum_r dgate[r]*readout[r]; gb_accum[0] and
 * gdb_accum[depth] += scale * sum_r dgate[r].  `workspace` holds
 * alodlm_gate_bwd_workspace(rows, hidden) floats. */
int64_t alodlm_gate_bwd_workspace(int64_t rows, int64_t hidden);
int alodlm_gate_bwd(const float* dgate, const void* readout, float scale, float* gw_accum,
                    float* gb_accum, float* gdb_accum, int64_t depth, int64_t rows,
                    int64_t hidden, float* workspace, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Optimizer (torch.nn.utils.clip_grad_norm_ and torch.optim.AdamW as called
 * at alodlm/train.py:49,140,143).  The tensor list is given by device arrays
 * of per-tensor pointers and numels and a chunk table: chunk c covers
 * elements [chunk_start[c], chunk_start[c] + chunk_size) of tensor
 * chunk_tensor[c].
 * grad_norm: total_norm[0] = sqrt(sum g^2); `partial` holds n_chunks floats.
 * adamw: decoupled decay p *= 1 - lr*wd[t], then Adam with bias correction
 * for `step` (>= 1) on the float master; m and v float; the dtype param is
 * rewritten from the master when it is a separate tensor.  If total_norm is
 * not NULL the gradient is scaled by min(1, max_norm/(total_norm+1e-6)),
 * read on the device.  grad_dtype is the gradients' storage type: `dtype`,
 * or ALODLM_F32 for float32 gradients of bf16 parameters (the step's
 * float32 gradient arena, read without a rounding to bf16).
 * ------------------------------------------------------------------------ */
int alodlm_grad_norm(const void* const* grads, const int32_t* chunk_tensor,
                     const int64_t* chunk_start, const int64_t* numels, int64_t n_chunks,
                     int64_t chunk_size, int dtype, float* partial, float* total_norm,
                     void* stream);
int alodlm_adamw(void* const* params, float* const* master, float* const* exp_avg,
                 float* const* exp_avg_sq, const void* const* grads,
                 const int32_t* chunk_tensor, const int64_t* chunk_start, const int64_t* numels,
                 const float* weight_decay, int64_t n_chunks, int64_t chunk_size,
                 const float* total_norm, float max_norm, float lr, float beta1, float beta2,
                 float eps, int64_t step, int dtype, int grad_dtype, void* stream);

/* Elementwise helpers. */
/* dst = cast(src * scale[0]); scale is a device scalar or null (no scaling).
 * Casts the float32 gradient arena to the parameter dtype for autograd,
 * applying the upstream gradient of the loss (torch's loss.backward() seed,
 * alodlm/train.py:136) without reading it on the host. */
int alodlm_cast_f32(const float* src, const float* scale, void* dst, int64_t n, int dtype,
                    void* stream);
int alodlm_scale_f32(float* x, const float* scale, int64_t n, void* stream);
/* x *= scale[0] in the storage dtype (scale is a device scalar), and the
 * float32 y = scale[0] * x + (accumulate ? y : 0) (scale may be NULL for 1).
 * The step computes the LM head's input and weight gradients in the forward,
 * where dL/dlogits is final at each depth, for a unit upstream gradient; the
 * backward applies torch's loss.backward() seed (alodlm/train.py:136,
 * alodlm/model.py:161 through torch.nn.Linear's backward) with these, without
 * reading it on the host. */
int alodlm_scale(void* x, const float* scale, int64_t n, int dtype, void* stream);
int alodlm_scale_add_f32(const float* x, float* y, int64_t n, const float* scale, int accumulate,
                         void* stream);
/* dst[c][r] = src[r][c] for a row-major rows x cols matrix (dst and src must
 * not overlap).  The step keeps transposed copies of the projection weights
 * ([in, out], refreshed at the start of every forward): the layers' forward
 * products run faster with the weight operand in out-contiguous rows (the
 * LM-head product reads the [out, in] weight itself, faster that way).  It
 * replaces the weight layout the forward products of alodlm/model.py:52-58
 * read through torch.nn.Linear. */
int alodlm_transpose(const void* src, void* dst, int64_t rows, int64_t cols, int dtype,
                     void* stream);
/* Stores 1 into *flag (never clears it) when any of the n elements of x is inf
 * or NaN; reads x once.  The step checks the LM-head weight with it, so that
 * the loss can follow the reference's 0 * sum(logits) term
 * (alodlm/model.py:186) without computing the logits of rows that carry no
 * loss. */
int alodlm_check_finite(const void* x, int64_t n, int dtype, int32_t* flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ALODLM_HIP_H */
