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
 * T == 1 runs the decode kernel; T > 1 runs the prefill path.
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
 * chunk_len: 0 = library default; otherwise the chunk length of the chunked
 * form (16, 32 or 64).
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

#ifdef __cplusplus
}
#endif

#endif /* RWKV7_HIP_H */
