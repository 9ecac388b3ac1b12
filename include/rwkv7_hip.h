/*
 * rwkv7_hip.h - C ABI of the gfx950 (MI355X) WKV7 decode / prefill / rollout library.
 *
 * Plain C: pointers are device pointers, sizes are element counts, `stream` is a
 * hipStream_t passed as void* (NULL = the default stream).  Every entry point
 * returns RWKV7_OK (0) or an error code and never throws; rwkv7_last_error()
 * gives the calling thread's last message.  Kernels are enqueued on `stream`
 * and nothing synchronises.  The library keeps no global state, so concurrent
 * calls on different streams are safe as long as they write disjoint memory.
 *
 * dtype codes: 0 = float32, 1 = float16, 2 = bfloat16 (the I/O type of
 * r, w, k, v, a, b, y).  The WKV state is always float32, layout
 * [slots][H][64][64], row = value index, column = key index
 * (rwkvtune/models/rwkv7/operators/cuda/wkv7s.cu:13).  Head size is 64.
 * `w` is the raw decay input: the kernels apply exp(-exp(w)) (wkv7s.cu:27).
 * Alignment: the WKV entry points (rwkv7s_forward, rwkv7_wkv_decode,
 * rwkv7_wkv_prefill) need r, w, k, v, a, b aligned to 4 elements (8 bytes for
 * 16-bit types, 16 for float32) and the state to 16 bytes; other pointers
 * return RWKV7_ERR_INVALID.  Fresh allocations always qualify.
 */
#ifndef RWKV7_HIP_H
#define RWKV7_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    RWKV7_DTYPE_F32 = 0,
    RWKV7_DTYPE_F16 = 1,
    RWKV7_DTYPE_BF16 = 2
};

enum {
    RWKV7_OK = 0,
    RWKV7_ERR_INVALID = 1,     /* bad size, null pointer or dtype */
    RWKV7_ERR_UNSUPPORTED = 2, /* valid request this build does not serve */
    RWKV7_ERR_LAUNCH = 3       /* the HIP runtime rejected a launch */
};

/* ABI version of this header (bumped on any signature change). */
int rwkv7_abi_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char *rwkv7_last_error(void);

/*
 * Stateful WKV7 over a dense batch: inputs and y are [B, T, C] (C = H*64),
 * state is [B, H, 64, 64] float32, updated in place.
 * Replaces torch.ops.wkv7s_custom.forward_{fp16,bf16,fp32}(B, T, C, H, state,
 * r, w, k, v, a, b, y) - rwkvtune/models/rwkv7/operators/cuda/wkv7s_op.cpp:8-30,
 * launched by cuda_forward_template (wkv7s.cu:56-62).  Differences: a dtype
 * code instead of three symbols, an explicit stream, and the precondition
 * C == H*64 (a host assert in the reference, wkv7s.cu:59) is an error return.
 * T == 1 runs the decode kernel; T > 1 runs the chunked prefill kernel.
 */
int rwkv7s_forward(int dtype, int64_t B, int64_t T, int64_t C, int64_t H,
                   float *state, const void *r, const void *w, const void *k,
                   const void *v, const void *a, const void *b, void *y,
                   void *stream);

/*
 * Single-token decode on a resident state pool.  Row s of the [B, C] inputs
 * and y belongs to pool slot slot_idx[s] (int32 device array; NULL = identity);
 * rows whose slot is negative or >= pool_slots are skipped (y untouched).
 * Replaces the per-layer call chain the reference's decode step makes through
 * load_wkv7_operator(...)(r, w, k, v, -kk, kk*a, state=att_kv, return_state=True)
 * (rwkvtune/models/rwkv7/model.py:229-250 -> wkv_loader.py:465-497), without the
 * gather/scatter of slot states around it (rwkvtune/inference/scheduler_core.py:377-395).
 */
int rwkv7_wkv_decode(int dtype, int64_t B, int64_t H, float *state_pool,
                     int64_t pool_slots, const int32_t *slot_idx,
                     const void *r, const void *w, const void *k, const void *v,
                     const void *a, const void *b, void *y, void *stream);

/*
 * Ragged prefill: nseq sequences packed as [total_tokens, C]; sequence s is
 * rows [cu_seqlens[s], cu_seqlens[s+1]) (int32 device array of nseq+1 entries,
 * non-decreasing, cu_seqlens[nseq] == total_tokens) and starts from pool slot
 * slot_idx[s] (NULL = identity), which receives its final state.  Malformed
 * rows (cu out of range, slot out of range or negative) are skipped.
 * chunk_len: 0, 16, 32 or 64 = the chunked MFMA form (contractions on bf16
 * matrix cores with hi/lo operand splitting, exact token-serial fallback for
 * chunks with a per-token log-decay below -1.25); it tiles by 32 tokens
 * whatever the value, which only names the caller's chunking and does not
 * change the result.  1 = the token-serial kernel.
 * Replaces the reference's chunked prefill, which calls the same token-serial
 * kernel once per length group and chunk (rwkvtune/inference/grpo_batch_generator.py:353-456,
 * scheduler_core.py:513-600 -> wkv7s.cu:22).
 */
int rwkv7_wkv_prefill(int dtype, int64_t nseq, int64_t H, int64_t total_tokens,
                      const int32_t *cu_seqlens, const int32_t *slot_idx,
                      float *state_pool, int64_t pool_slots,
                      const void *r, const void *w, const void *k, const void *v,
                      const void *a, const void *b, void *y, int chunk_len,
                      void *stream);

/*
 * Training operator: replaces torch.ops.wind_backstepping.forward / backward
 * (rwkvtune/models/rwkv7/operators/cuda/wkv7_op.cpp:6-18, kernels
 * wkv7_cuda.cu:10-142) and, with s0 / ds_in / ds0, the infinite-context op
 * (wkv7_infctx_op.cpp, wkv7_infctx_cuda.cu:24-305).  Inputs r, w (raw: the
 * decay is exp(-exp(w))), k, v, a, b, y, dy and the gradients are [B, T, H, 64]
 * in the I/O dtype (any T >= 1; the standard op's caller requires T % 16 == 0).
 *
 * forward: y; sa = S_{t-1} a_t (float32 [B, T, H, 64]); ckpt = the float32 state
 * [64][64] (row = value index) after every 16th token and after the last one,
 * [B, H, ceil(T/16), 64, 64] (rwkv7_wkv_train_ckpt_floats floats, 16-byte
 * aligned).  s0: initial state [B, H, 64, 64] float32 (NULL: zero); s_out
 * (nullable, may alias s0) receives the final state.  16-bit inputs aligned to
 * 4 elements run in 32-token chunks on the matrix cores (float32-accumulated
 * hi / lo bf16 operand parts); float32 or unaligned inputs token by token.
 * backward: from dy and the forward's ckpt and sa, the gradients dr, dw (w.r.t.
 * the raw w), dk, dv, da, db; ds_in (nullable) is the gradient of the final
 * state, ds0 (nullable) receives the initial state's.  The state is stepped
 * back one token at a time from the checkpoints (S_{t-1} = (S_t - v k^T -
 * sa b^T) / w~, as the reference), so it needs w~ = exp(-exp(w)) > 0.
 */
int64_t rwkv7_wkv_train_ckpt_floats(int64_t B, int64_t T, int64_t H);
int rwkv7_wkv_train_forward(int dtype, int64_t B, int64_t T, int64_t H, const void *r,
                            const void *w, const void *k, const void *v, const void *a,
                            const void *b, void *y, const float *s0, float *s_out,
                            float *ckpt, float *sa, void *stream);
int rwkv7_wkv_train_backward(int dtype, int64_t B, int64_t T, int64_t H, const void *r,
                             const void *w, const void *k, const void *v, const void *a,
                             const void *b, const void *dy, const float *ckpt,
                             const float *sa, const float *ds_in, void *dr, void *dw,
                             void *dk, void *dv, void *da, void *db, float *ds0,
                             void *stream);

/* ------------------------------------------------------------------------
 * Layer kernels of the stateful model forward.  They replace the eager torch
 * op chains of RWKV7Block / RWKV7TimeMix / RWKV7ChannelMix.forward_with_state
 * (rwkvtune/models/rwkv7/model.py:174-418); the dense projections between
 * them are plain library GEMMs.  Rows are token positions of a packed batch;
 * the rows of one sequence are contiguous.  row_slot[m] = pool slot of row m's
 * sequence (negative: no state, x_prev = 0, nothing written).  row_last[m] >= 0
 * marks the first row of a sequence in this call and holds the index of the
 * sequence's last row; -1 on every other row.  Small per-channel parameters
 * are float32; activations use `dtype`.  C <= 8000 and a multiple of 4; H a
 * multiple of 4; n_mix is 1, 6 or 7.
 * ------------------------------------------------------------------------ */

/*
 * Residual source + LayerNorm + token shift + lerps.  The residual of row m is
 * emb[tokens[m]] (tokens non-null) or x_in[m] (+ add[m] when add is non-null),
 * then ln0 when ln0_w is non-null.  add_parts = 0: add is [M, C] in the I/O
 * dtype.  add_parts = P >= 1 (not with tokens): add is float32 partial sums,
 * plane q at add + q * add_part_stride floats (16-byte aligned, stride a multiple
 * of 4 and >= M * C), and add[m] is the in-order sum of the P planes' row m
 * rounded to the I/O dtype - the output of rwkv7_gemm_decode_partials, which
 * this consumes in place of the split-K reduction; it is written to x_out (nullable, float32
 * [M, C]).  h = LayerNorm(residual; ln_w, ln_b, eps 1e-5); h_prev is the previous
 * row's h, or prev_pool[slot] on a sequence's first row; out[j][m] =
 * h + (h_prev - h) * mix[j] for j < n_mix (out: [n_mix, M, C]).  The sequence's
 * last h is stored to prev_pool[slot] (float32 [pool_slots, C]).
 * Replaces model.py:393-398 (ln0, ln1), 196-208 (shift + six lerps) and 412
 * (att_x_prev), and with n_mix = 1 model.py:406-407, 315-321 (ln2, FFN shift).
 */
int rwkv7_shift_mix(int dtype, int64_t M, int64_t C, const float *x_in, const void *add,
                    int add_parts, int64_t add_part_stride,
                    const int64_t *tokens, const void *emb, int64_t vocab,
                    const float *ln0_w, const float *ln0_b, float *x_out,
                    const float *ln_w, const float *ln_b, float *prev_pool,
                    int64_t pool_slots, const int32_t *row_slot, const int32_t *row_last,
                    int n_mix, const float *mix, void *out, void *stream);

/* out[n] = LayerNorm(x_in[rows[n]] + add[rows[n]]) (rows NULL: row n; add nullable;
 * add_parts / add_part_stride as for rwkv7_shift_mix, stride >= C).
 * Replaces ln_out (model.py:494) restricted to the rows whose logits are used. */
int rwkv7_final_norm(int dtype, int64_t n, int64_t C, const float *x_in, const void *add,
                     int add_parts, int64_t add_part_stride, const int32_t *rows,
                     const float *ln_w, const float *ln_b, void *out, void *stream);

/* In-place element-wise activation of n elements: kind 0 = tanh (decay LoRA,
 * model.py:211), 1 = sigmoid (gate LoRA, model.py:221), 2 = relu(x)^2 (FFN,
 * model.py:337). */
int rwkv7_activation(int dtype, int kind, int64_t n, void *x, void *stream);

/*
 * params: 8 float32 [C] vectors w0, a0, v0 (NULL on layer 0), k_k, k_a, r_k
 * (the [H, N] tensor flattened), ln_x weight, ln_x bias.
 *
 * rwkv7_tmix_prep: from the projection outputs r, k, v and the LoRA outputs
 * (w_lora = tanh(xw@w1)@w2, a_lora = (xa@a1)@a2, v_lora = (xv@v1)@v2), write the
 * six WKV operands wkv_ops = {r, w_raw, k', v', -kk, kk*a} ([M, C] each, in the
 * I/O dtype: the reference hands its WKV kernel tensors of the model dtype) and,
 * on layer 0, v_first = v (float32 [M, C]; read on later layers).  wkv_ops[0]
 * may be NULL: r is then not copied and the caller hands r itself to the WKV op.
 * Replaces model.py:215-227 and the operand construction of model.py:233-247.
 */
int rwkv7_tmix_prep(int dtype, int64_t M, int64_t H, int layer0, const void *r, const void *k,
                    const void *v, const void *w_lora, const void *a_lora, const void *v_lora,
                    float *v_first, const float *const *params, void *const *wkv_ops,
                    void *stream);

/* out = (GroupNorm_H(y; ln_x, eps 64e-5) + sum_head(r*k'*r_k) * v') * g, from the
 * WKV output y and the operands written by rwkv7_tmix_prep (all in the I/O dtype).
 * Replaces model.py:258-269 (before the output projection). */
int rwkv7_tmix_post(int dtype, int64_t M, int64_t H, const void *y, const void *r_op,
                    const void *k_op, const void *v_op, const void *g,
                    const float *const *params, void *out, void *stream);

/* Single-token fused path: rwkv7_tmix_prep + one WKV step on
 * state_pool[row_slot[m]] (float32 [pool_slots, H, 64, 64], in place) +
 * rwkv7_tmix_post, one four-wave block per (row, head).  Rows with a negative slot get
 * out = 0 and touch no state.  Replaces model.py:215-269 for T = 1 together
 * with the decode call of the WKV operator (model.py:229-250 -> wkv7s.cu:5-54). */
int rwkv7_tmix_decode(int dtype, int64_t M, int64_t H, int layer0, const void *r, const void *k,
                      const void *v, const void *w_lora, const void *a_lora, const void *v_lora,
                      const void *g, float *v_first, const float *const *params,
                      float *state_pool, int64_t pool_slots, const int32_t *row_slot,
                      void *out, void *stream);

/*
 * Grouped bf16 GEMM for decode-sized projections (M up to a few hundred rows):
 * `count` (1..8) independent problems in one launch, problem i computing
 *   C_i[M, N_i] = epi_i(A_i[M, K_i] . B_i^T)
 * with A_i, C_i bf16 row-major (row strides lda_i, ldc_i) and B_i the
 * nn.Linear weight [N_i][K_i] in the packed layout of rwkv7_gemm_pack, float32
 * accumulation.  epi: 0 none, 1 relu(x)^2, 2 tanh, 3 sigmoid.  K_i % 8 == 0,
 * lda_i % 8 == 0 and >= K_i, A_i and B_i 16-byte aligned.  The pointer and
 * size arrays are host arrays of `count` entries.  Problems whose K is split
 * across blocks write float32 partial rows to `workspace` (contents need no
 * initialisation) and a second launch on `stream` reduces them;
 * rwkv7_gemm_decode_workspace gives the floats a problem set needs (-1 on
 * invalid sizes).  Calls that share a workspace must not overlap.  Replaces
 * the decode step's projection chain of model.py:210-221, 269, 337-338, 495
 * (torch nn.Linear / matmul calls and the tanh / sigmoid / relu^2 between them).
 */
int64_t rwkv7_gemm_decode_workspace(int64_t M, int count, const int *N, const int *K);
int rwkv7_gemm_decode(int64_t M, int count, const void *const *A, const void *const *B,
                      void *const *C, const int64_t *lda, const int64_t *ldc,
                      const int *N, const int *K, const int *epi,
                      float *workspace, int64_t workspace_floats, void *stream);

/*
 * rwkv7_gemm_decode without a workspace argument and without any allocation:
 * split-K partials go to the library's static scratch, a fixed array of
 * RWKV7_GEMM_SCRATCH_FLOATS floats (8 MiB) that every GPU the library runs on
 * holds until the process ends.  Problem sets needing more (see
 * rwkv7_gemm_decode_workspace) return RWKV7_ERR_INVALID; with the library's
 * split plan none does: K is split only at M <= 32 rows, to about 256 blocks of
 * at most 32 x 32 outputs, so a set needs at most 510 * 32 * 32 = 522,240
 * floats.  The check stays for plans that may split more.  The scratch needs no clearing
 * (every range writes all its partials before they are read).  All calls on one
 * GPU share its scratch, so calls that overlap on one GPU (concurrent streams,
 * threads) race; calls in one stream's order do not.  The first call on a device
 * looks up that device's scratch address once.
 * No counterpart in the reference: this entry point is for callers that cannot
 * allocate device memory - code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  Results equal rwkv7_gemm_decode's bit for bit.
 */
#define RWKV7_GEMM_SCRATCH_FLOATS (1 << 21)
int rwkv7_gemm_decode_noalloc(int64_t M, int count, const void *const *A, const void *const *B,
                              void *const *C, const int64_t *lda, const int64_t *ldc,
                              const int *N, const int *K, const int *epi, void *stream);

/*
 * One problem of rwkv7_gemm_decode (epi 0) without its reduction: the products
 * of the plan's P = rwkv7_gemm_decode_partial_count(M, N, K) K ranges are left in
 * `workspace` as float32 planes [P][M][N] (16-byte aligned, P * M * N floats),
 * and *parts (host) receives P (also when P = 1).  Their in-order sum rounded to
 * bf16 is the product (rwkv7_gemm_decode may split K differently, so its C can
 * differ in the last bit); rwkv7_shift_mix / rwkv7_final_norm take the
 * planes directly (add_parts = P, add_part_stride = M * N), which saves the
 * reduction launch.  For the FFN value projection (model.py:338) ahead of the
 * next layer's residual add.  partial_count returns -1 on invalid sizes.
 */
int rwkv7_gemm_decode_partial_count(int64_t M, int N, int K);
int rwkv7_gemm_decode_partials(int64_t M, const void *A, const void *B, int64_t lda, int N, int K,
                               float *workspace, int64_t workspace_floats, int32_t *parts,
                               void *stream);

/*
 * Weight packing for rwkv7_gemm_decode: B [N][K] bf16 (row stride ldb, a
 * multiple of 8, K % 8 == 0) into rwkv7_gemm_packed_elems(N, K) bf16 elements
 * at `out`: 64 x 64 tiles of 8 KB, tile (nt, kt) at element
 * (nt * ceil(K/64) + kt) * 4096, rows past N and columns past K zero, the 16-byte
 * chunks of a tile row in the order the GEMM's LDS stage uses.  Run once per
 * weight (no counterpart in the reference: its weights are read in place).
 * rwkv7_gemm_packed_elems returns -1 on invalid sizes.
 */
int64_t rwkv7_gemm_packed_elems(int N, int K);
int rwkv7_gemm_pack(const void *B, int64_t ldb, int N, int K, void *out, void *stream);

/*
 * LM head for decode rows: logits[M, V] (bf16, row stride ldc) = A[M, K] . W^T
 * with A bf16 row-major (row stride lda) and W the head weight [V][K] in the
 * packed layout of rwkv7_head_pack, float32 accumulation rounded to bf16 once.
 * V % 256 == 0, K % 64 == 0 and 256 <= K <= 65536; lda >= K and ldc >= V, both
 * multiples of 8; A, the packed weight and the logits 16-byte aligned.  One
 * block per 256 columns streams its rows of W once per row tile; rows are tiled
 * by 64 (M <= 64) or 128, so any M works, but above 128 rows W is streamed
 * once per 128 rows (a library GEMM with 256-row tiles is faster there).
 * Replaces the head of the decode step, model.py:494-495 (self.head on the
 * normalised last hidden state).
 */
int rwkv7_head_logits(int64_t M, int V, int K, const void *A, int64_t lda, const void *W_packed,
                      void *logits, int64_t ldc, void *stream);

/*
 * Weight packing for rwkv7_head_logits: W [V][K] bf16 (row stride ldw, a
 * multiple of 8, K % 64 == 0) into rwkv7_head_packed_elems(V, K) bf16
 * elements: 64-row x 32-column pieces of 4 KB, piece (g, kt) at element
 * (g * K/32 + kt) * 2048 holding rows 64 g .. 64 g + 63, columns 32 kt ..
 * 32 kt + 31 row-major; rows past V zero.  Run once per weight (no counterpart
 * in the reference: its head weight is read in place).
 * rwkv7_head_packed_elems returns -1 on invalid sizes.
 */
int64_t rwkv7_head_packed_elems(int V, int K);
int rwkv7_head_pack(const void *W, int64_t ldw, int V, int K, void *out, void *stream);

/* ------------------------------------------------------------------------
 * Sampling
 * ------------------------------------------------------------------------ */

/*
 * One token per row of logits [M, V] (row stride ld >= V, V <= 65536, dtype of
 * the logits) into out_tok (int64 [M]) and out_logp (float32 [M]).  Per row:
 * temperature[m] (< 1e-6: greedy), top_p[m], top_k[m] (0 = off); ids above
 * max_valid_id are banned (negative: no ban).  Optional logit bias in CSR form:
 * bias_ids / bias_val [bias_off[m] .. bias_off[m+1]) (bias_off NULL: none).
 * active (uint8 [M], nullable): rows with 0 are skipped.  Draws use a
 * counter-based hash of (seed, rng_key[m], rng_ctr[m]).  rule 1 =
 * TokenSampler.sample (rwkvtune/inference/core.py:40-137), rule 0 =
 * TokenSampler.sample_batch (core.py:142-236), rule 2 =
 * GenerationMixin.generate (rwkvtune/models/generation_mixin.py:180-211:
 * top-k, then top-p only when 0 < top_p < 1, keeping the crossing token); see
 * sampler.hip for the exact rules.  Replaces both methods' torch op chains (softmax, sort, cumsum,
 * multinomial, gather) and their per-sequence .item() synchronisations.
 */
int rwkv7_sample(int dtype, int64_t M, int64_t V, const void *logits, int64_t ld, int rule,
                 int64_t max_valid_id, const float *temperature, const float *top_p,
                 const int32_t *top_k, const int32_t *bias_off, const int32_t *bias_ids,
                 const float *bias_val, const uint8_t *active, uint64_t seed,
                 const int64_t *rng_key, const int32_t *rng_ctr, int64_t *out_tok,
                 float *out_logp, void *stream);

/*
 * In-place repetition penalty on float32 logits [M, V] (row stride ld): for
 * every occurrence of an id in row m's history, logit / penalty if logit > 0
 * else logit * penalty.  History of row m: hist[hist_start[m] .. + hist_len[m])
 * then, when hist2 is non-NULL, hist2[hist2_start[m] .. + hist2_len[m]).
 * penalty == 1 or <= 0 is a no-op.  Replaces _apply_repetition_penalty
 * (rwkvtune/inference/grpo_batch_generator.py:25-42).
 */
int rwkv7_repetition_penalty(int64_t M, int64_t V, float *logits, int64_t ld, float penalty,
                             const int32_t *hist, const int64_t *hist_start, const int32_t *hist_len,
                             const int32_t *hist2, const int64_t *hist2_start,
                             const int32_t *hist2_len, const uint8_t *active, void *stream);

/* ------------------------------------------------------------------------
 * GPU slot table of the rollout.  Replaces the Python bookkeeping of the
 * reference's decode loops - active-sequence lists, EOS / length retirement,
 * admission of waiting sequences into free slots and the per-step state
 * gather / scatter (rwkvtune/inference/grpo_batch_generator.py:458-610,
 * rwkvtune/inference/scheduler_core.py:250-299, 363-395, 445-511) - so decode
 * steps run back to back with no host round trip.
 *
 * Device tables (n sequences, S slots, maxlen token columns):
 *   seq_prompt[n] int32   index of the sequence's prompt state in the store
 *   seq_max_new[n] int32  token cap;  seq_ngen[n] int32  tokens so far
 *   seq_done[n] uint8;    out_tok / out_logp / out_step [n, maxlen]
 *                         (int32 / float32 / int32: token, its sampling
 *                         log-probability, the decode step that made it)
 *   slot_seq[S] int32     sequence in the slot, -1 = free
 *   row_slot[S] int32     slot of row r or -1: the row_slot of the model kernels
 *   tok_in[S] int64       next input token of row r
 *   slot_row[S] int32     (optional, compaction) row of slot s, -1 = free
 *   counters[5] int32     next waiting sequence, finished sequences, decode
 *                         steps committed, admissions of the current step, live
 *                         rows (with compaction)
 *   admit_slot / admit_src [S] int32: this step's admissions (slot <- store entry)
 * Rows are what a decode step computes; slots hold the state.  Without
 * compaction row r is slot r.  With it, the live slots take rows 0 .. live-1 in
 * slot order and rows past them are -1, so a step may run only a leading bucket
 * of rows that covers the live ones.
 * ------------------------------------------------------------------------ */

/* Record each sequence's first token (sampled from its prompt's last logits):
 * out_tok[q][0] = tok[q], seq_ngen[q] = 1; with first_can_finish, EOS (eos >= 0)
 * or a cap of 1 finishes the sequence (SchedulerCore); without it the first
 * token never does (GRPOBatchGenerator, grpo_batch_generator.py:283-285). */
int rwkv7_rollout_first(int64_t n, int64_t maxlen, const int64_t *tok, const float *logp,
                        const int32_t *seq_max_new, int32_t *seq_ngen, uint8_t *seq_done,
                        int32_t *out_tok, float *out_logp, int32_t *out_step, int64_t eos,
                        int first_can_finish, int32_t *counters, void *stream);

/* Prefill in the slot: record the first tokens of the m sequences seq_idx[i]
 * (tok[i] / logp[i], sampled from the logits of their prompts' last tokens once
 * the prompts were prefilled into their slots), as rwkv7_rollout_first does for
 * all n; indices outside [0, n) are skipped.  The next rwkv7_rollout_commit gives
 * each such slot a row fed with that token, or frees it when the first token
 * finished the sequence.  With the commit's rule that a slot whose sequence has
 * no token yet holds no row, this is the reference SchedulerCore's "admit into a
 * free slot, prefill there, then decode" (rwkvtune/inference/scheduler_core.py:
 * 250-299, 513-600) without a host read of each step's tokens. */
int rwkv7_rollout_activate(int64_t m, const int32_t *seq_idx, int64_t n, int64_t maxlen,
                           const int64_t *tok, const float *logp, const int32_t *seq_max_new,
                           int32_t *seq_ngen, uint8_t *seq_done, int32_t *out_tok, float *out_logp,
                           int32_t *out_step, int64_t eos, int first_can_finish, int32_t *counters,
                           void *stream);

/* One block: with have_sample, append tok[r] / logp[r] of the row r the slot
 * ran in to the sequence in slot s, finish it on EOS or its cap; then every free
 * slot (or slot whose sequence finished at its first token) takes the next
 * waiting, unfinished sequence (index order) and lists the state copy it needs;
 * finally the row table is rebuilt over the live slots - those whose sequence
 * has at least one token (compacted when slot_row is non-NULL; slot_row must
 * then start as all -1 with every slot free).  S <= 1024. */
int rwkv7_rollout_commit(int64_t S, int64_t n, int64_t maxlen, int have_sample, const int64_t *tok,
                         const float *logp, int32_t *slot_seq, int32_t *row_slot, int32_t *slot_row,
                         int64_t *tok_in,
                         const int32_t *seq_prompt, const int32_t *seq_max_new, int32_t *seq_ngen,
                         uint8_t *seq_done, int32_t *out_tok, float *out_logp, int32_t *out_step,
                         int64_t eos, int32_t *counters, int32_t *admit_slot, int32_t *admit_src,
                         void *stream);

/* Per-row sampler inputs of the step for rows 0 .. S-1 (row r holds slot
 * row_slot[r]; row_slot NULL: row r is slot r): active[r], rng_key[r] =
 * seq_key[q] of the row's sequence q (seq_key NULL: q), rng_ctr[r] = its
 * position; optionally (hist_start non-NULL) the two history segments of the
 * repetition penalty (prompt ids in a packed prompt array at prompt_start[p] /
 * prompt_len[p]; generated ids in out_tok), and optionally (seq_temp non-NULL)
 * per-sequence temperature / top_p / top_k copied to the row. */
int rwkv7_rollout_prepare(int64_t S, int64_t maxlen, const int32_t *row_slot, const int32_t *slot_seq,
                          const int64_t *seq_key, const int32_t *seq_ngen,
                          const int32_t *seq_prompt, const int64_t *prompt_start,
                          const int32_t *prompt_len, uint8_t *active, int64_t *rng_key,
                          int32_t *rng_ctr, int64_t *hist_start, int32_t *hist_len,
                          int64_t *hist2_start, int32_t *hist2_len, const float *seq_temp,
                          const float *seq_top_p, const int32_t *seq_top_k, float *temp,
                          float *top_p, int32_t *top_k, void *stream);

/* Fork-on-admit: copy every layer's state (kv [L][U or S][kv_elems], att_x /
 * ffn_x [L][U or S][C], float32) of store entry admit_src[i] into slot
 * admit_slot[i], for the counters[3] admissions of the step.  Replaces the
 * index copies of grpo_batch_generator.py:233-260 and the slot reset / load of
 * scheduler_core.py:301-350. */
int rwkv7_admit_copy(const int32_t *counters, const int32_t *admit_slot, const int32_t *admit_src,
                     int64_t L, int64_t S, int64_t U, int64_t kv_elems, int64_t C,
                     const float *src_kv, const float *src_ax, const float *src_fx,
                     float *dst_kv, float *dst_ax, float *dst_fx, void *stream);

/* ------------------------------------------------------------------------
 * Log-probabilities of chosen tokens
 * ------------------------------------------------------------------------ */

/*
 * out[r] = log_softmax(logits[r, :V])[index[r]] for R rows of logits (row
 * stride ld >= V, `dtype`), written in the logits' dtype: float32 rows give
 * x[i] - logsumexp(x); bf16 / fp16 rows give x[i] - lse with lse the float32
 * logsumexp rounded to the dtype, subtracted and rounded in the dtype.  index is
 * int64 [R]; an index outside [0, V) gives NaN.  Replaces selective_log_softmax
 * (rwkvtune/training/grpo/utils.py:13-103) as used by the GRPO log-prob
 * recompute (grpo/lightning_module.py:1810-1964).
 */
int rwkv7_selective_log_softmax(int dtype, int64_t R, int64_t V, const void *logits, int64_t ld,
                                const int64_t *index, void *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV7_HIP_H */
