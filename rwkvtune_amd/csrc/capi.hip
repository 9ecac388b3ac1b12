// C ABI entry points (declared in include/rwkv7_hip.h): argument checks, dtype
// dispatch and launches.  No exceptions cross this boundary.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"
#include "rwkv7_hip.h"

template <typename IO>
hipError_t launch_wkv7_seq(int nseq, int H, int T_uniform, const int32_t* cu_seqlens,
                           const int32_t* slot_idx, int pool_slots, int total_tokens,
                           float* state, const void* r, const void* w, const void* k,
                           const void* v, const void* a, const void* b, void* y,
                           hipStream_t stream);

template <typename IO>
hipError_t launch_wkv7_chunk(int nseq, int H, int T_uniform, const int32_t* cu_seqlens, const int32_t* slot_idx,
                             int pool_slots, int total_tokens, float* state, const void* r, const void* w,
                             const void* k, const void* v, const void* a, const void* b, void* y, hipStream_t stream);

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = '\0';
    return RWKV7_OK;
}

int launch_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(RWKV7_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool dtype_ok(int dtype) {
    return dtype == RWKV7_DTYPE_F32 || dtype == RWKV7_DTYPE_F16 || dtype == RWKV7_DTYPE_BF16;
}

constexpr int64_t kMaxInt = 0x7fffffff;

int seq_dispatch(int dtype, int nseq, int H, int T_uniform, const int32_t* cu, const int32_t* slot,
                 int pool_slots, int total, float* state, const void* r, const void* w,
                 const void* k, const void* v, const void* a, const void* b, void* y,
                 hipStream_t st) {
    hipError_t e;
    switch (dtype) {
        case RWKV7_DTYPE_F32:
            e = launch_wkv7_seq<float>(nseq, H, T_uniform, cu, slot, pool_slots, total, state,
                                       r, w, k, v, a, b, y, st);
            break;
        case RWKV7_DTYPE_F16:
            e = launch_wkv7_seq<f16_t>(nseq, H, T_uniform, cu, slot, pool_slots, total, state,
                                       r, w, k, v, a, b, y, st);
            break;
        default:
            e = launch_wkv7_seq<bf16_t>(nseq, H, T_uniform, cu, slot, pool_slots, total, state,
                                        r, w, k, v, a, b, y, st);
            break;
    }
    return launch_status(e, "wkv7_seq_kernel");
}

int chunk_dispatch(int dtype, int nseq, int H, int T_uniform, const int32_t* cu, const int32_t* slot, int pool_slots,
                   int total, float* state, const void* r, const void* w, const void* k, const void* v,
                   const void* a, const void* b, void* y, hipStream_t st) {
    hipError_t e;
    switch (dtype) {
        case RWKV7_DTYPE_F32:
            e = launch_wkv7_chunk<float>(nseq, H, T_uniform, cu, slot, pool_slots, total, state, r, w, k, v, a, b, y,
                                         st);
            break;
        case RWKV7_DTYPE_F16:
            e = launch_wkv7_chunk<f16_t>(nseq, H, T_uniform, cu, slot, pool_slots, total, state, r, w, k, v, a, b, y,
                                         st);
            break;
        default:
            e = launch_wkv7_chunk<bf16_t>(nseq, H, T_uniform, cu, slot, pool_slots, total, state, r, w, k, v, a, b,
                                          y, st);
            break;
    }
    return launch_status(e, "wkv7_chunk_kernel");
}

bool any_null(const void* p0, const void* p1, const void* p2, const void* p3, const void* p4,
              const void* p5, const void* p6, const void* p7) {
    return !p0 || !p1 || !p2 || !p3 || !p4 || !p5 || !p6 || !p7;
}

// The WKV kernels read 4 consecutive input elements per access (8 bytes for
// 16-bit types, 16 for float32) and the state 16 bytes at a time.
bool misaligned(int dtype, const void* state, const void* r, const void* w, const void* k, const void* v,
                const void* a, const void* b) {
    const uintptr_t m = dtype == RWKV7_DTYPE_F32 ? 15 : 7;
    return (((uintptr_t)r | (uintptr_t)w | (uintptr_t)k | (uintptr_t)v | (uintptr_t)a | (uintptr_t)b) & m) != 0 ||
           ((uintptr_t)state & 15) != 0;
}

}  // namespace

extern "C" int rwkv7_abi_version(void) { return 2; }

extern "C" const char* rwkv7_last_error(void) { return g_err; }

extern "C" int rwkv7s_forward(int dtype, int64_t B, int64_t T, int64_t C, int64_t H, float* state,
                              const void* r, const void* w, const void* k, const void* v,
                              const void* a, const void* b, void* y, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: bad dtype code %d", dtype);
    if (B < 0 || T < 0 || H <= 0) return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: bad sizes B=%lld T=%lld H=%lld",
                                              (long long)B, (long long)T, (long long)H);
    if (C != H * RWKV7_HEAD)
        return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: C=%lld != H*64 (H=%lld)", (long long)C, (long long)H);
    if (B == 0 || T == 0) return ok();
    // the token-serial kernel runs four blocks per (sequence, head)
    if (B * T > kMaxInt || 4 * B * H > kMaxInt || B * T * C > (int64_t)1 << 40)
        return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: problem too large");
    if (any_null(state, r, w, k, v, a, b, y)) return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: null pointer");
    if (misaligned(dtype, state, r, w, k, v, a, b))
        return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: inputs must be aligned to 4 elements, the state to 16 bytes");
    hipStream_t st = (hipStream_t)stream;
    if (T == 1)
        return seq_dispatch(dtype, (int)B, (int)H, 1, nullptr, nullptr, (int)B, (int)B, state, r, w, k, v, a, b, y, st);
    return chunk_dispatch(dtype, (int)B, (int)H, (int)T, nullptr, nullptr, (int)B, (int)(B * T), state, r, w, k, v, a,
                          b, y, st);
}

extern "C" int rwkv7_wkv_decode(int dtype, int64_t B, int64_t H, float* state_pool, int64_t pool_slots,
                                const int32_t* slot_idx, const void* r, const void* w, const void* k,
                                const void* v, const void* a, const void* b, void* y, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: bad dtype code %d", dtype);
    if (B < 0 || H <= 0 || pool_slots < 0)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: bad sizes B=%lld H=%lld slots=%lld", (long long)B,
                    (long long)H, (long long)pool_slots);
    if (B == 0) return ok();
    if (slot_idx == nullptr && pool_slots < B)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: identity slots need pool_slots >= B");
    if (4 * B * H > kMaxInt || pool_slots > kMaxInt) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: too large");
    if (any_null(state_pool, r, w, k, v, a, b, y)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: null pointer");
    if (misaligned(dtype, state_pool, r, w, k, v, a, b))
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: inputs must be aligned to 4 elements, the state to 16 bytes");
    return seq_dispatch(dtype, (int)B, (int)H, 1, nullptr, slot_idx, (int)pool_slots, (int)B, state_pool, r, w,
                        k, v, a, b, y, (hipStream_t)stream);
}

extern "C" int rwkv7_wkv_prefill(int dtype, int64_t nseq, int64_t H, int64_t total_tokens,
                                 const int32_t* cu_seqlens, const int32_t* slot_idx, float* state_pool,
                                 int64_t pool_slots, const void* r, const void* w, const void* k,
                                 const void* v, const void* a, const void* b, void* y, int chunk_len,
                                 void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: bad dtype code %d", dtype);
    if (nseq < 0 || H <= 0 || total_tokens < 0 || pool_slots < 0)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: bad sizes");
    if (chunk_len != 0 && chunk_len != 1 && chunk_len != 16 && chunk_len != 32 && chunk_len != 64)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: chunk_len must be 0, 1, 16, 32 or 64 (got %d)", chunk_len);
    if (nseq == 0 || total_tokens == 0) return ok();
    if (cu_seqlens == nullptr) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: cu_seqlens is required");
    if (slot_idx == nullptr && pool_slots < nseq)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: identity slots need pool_slots >= nseq");
    if (4 * nseq * H > kMaxInt || total_tokens > kMaxInt || pool_slots > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: too large");
    if (any_null(state_pool, r, w, k, v, a, b, y)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: null pointer");
    if (misaligned(dtype, state_pool, r, w, k, v, a, b))
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: inputs must be aligned to 4 elements, the state to 16 bytes");
    if (chunk_len == 1)
        return seq_dispatch(dtype, (int)nseq, (int)H, 0, cu_seqlens, slot_idx, (int)pool_slots, (int)total_tokens,
                            state_pool, r, w, k, v, a, b, y, (hipStream_t)stream);
    return chunk_dispatch(dtype, (int)nseq, (int)H, 0, cu_seqlens, slot_idx, (int)pool_slots, (int)total_tokens,
                          state_pool, r, w, k, v, a, b, y, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Layer kernels (rwkv7_layer.hip)
// ---------------------------------------------------------------------------

template <typename IO>
hipError_t launch_shift_mix(int M, int C, const float* x_in, const void* add, int add_parts, int64_t part_stride,
                            const int64_t* tokens, const void* emb, int64_t vocab, const float* ln0_w,
                            const float* ln0_b, float* x_out, const float* ln_w, const float* ln_b,
                            float* prev_pool, int pool_slots, const int32_t* row_slot, const int32_t* row_last,
                            int n_mix, const float* mix, void* out, hipStream_t st);
template <typename IO>
hipError_t launch_final_norm(int n, int C, const float* x_in, const void* add, int add_parts, int64_t part_stride,
                             const int32_t* rows, const float* ln_w, const float* ln_b, void* out, hipStream_t st);
template <typename IO>
hipError_t launch_activation(int kind, int64_t n, void* x, hipStream_t st);
template <typename IO>
hipError_t launch_tmix_prep(int M, int H, int layer0, const void* r, const void* k, const void* v,
                            const void* wl, const void* al, const void* vl, float* vfirst,
                            const float* const* params, void* const* ops, hipStream_t st);
template <typename IO>
hipError_t launch_tmix_post(int M, int H, const void* y, const void* r_op, const void* k_op,
                            const void* v_op, const void* g, const float* const* params, void* out,
                            hipStream_t st);
template <typename IO>
hipError_t launch_tmix_decode(int M, int H, int layer0, const void* r, const void* k, const void* v,
                              const void* wl, const void* al, const void* vl, const void* g,
                              float* vfirst, const float* const* params, float* state, int pool_slots,
                              const int32_t* row_slot, void* out, hipStream_t st);

#define RWKV7_DISPATCH(dtype, call)                         \
    switch (dtype) {                                        \
        case RWKV7_DTYPE_F32: { typedef float IO; e = call; break; }  \
        case RWKV7_DTYPE_F16: { typedef f16_t IO; e = call; break; }  \
        default: { typedef bf16_t IO; e = call; break; }    \
    }

namespace {
constexpr int64_t kMaxC = 8000;  // two fp32 rows of LDS per block
bool bad_c(int64_t C) { return C <= 0 || C > kMaxC; }
bool bad_h(int64_t H) { return H <= 0 || (H % 4) != 0 || H * RWKV7_HEAD > kMaxC; }
constexpr int kMaxAddParts = 64;
// add_parts > 0: `add` is float32 partial sums, 16-byte aligned, planes
// part_stride floats apart (a multiple of 4, at least min_stride)
bool bad_parts(int add_parts, const void* add, int64_t part_stride, int64_t min_stride) {
    if (add_parts == 0) return false;
    return add_parts < 0 || add_parts > kMaxAddParts || add == nullptr || (((uintptr_t)add) & 15) != 0 ||
           (add_parts > 1 && (part_stride < min_stride || (part_stride % 4) != 0));
}
}  // namespace

extern "C" int rwkv7_shift_mix(int dtype, int64_t M, int64_t C, const float* x_in, const void* add,
                               int add_parts, int64_t add_part_stride,
                               const int64_t* tokens, const void* emb, int64_t vocab,
                               const float* ln0_w, const float* ln0_b, float* x_out,
                               const float* ln_w, const float* ln_b, float* prev_pool,
                               int64_t pool_slots, const int32_t* row_slot, const int32_t* row_last,
                               int n_mix, const float* mix, void* out, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_shift_mix: bad dtype code %d", dtype);
    if (M < 0 || bad_c(C) || (C % 4) != 0 || (n_mix != 1 && n_mix != 6 && n_mix != 7) || pool_slots < 0 ||
        M > kMaxInt)
        return fail(RWKV7_ERR_INVALID,
                    "rwkv7_shift_mix: bad sizes M=%lld C=%lld n_mix=%d (C %% 4 == 0, n_mix 1, 6 or 7)",
                    (long long)M, (long long)C, n_mix);
    if (M == 0) return ok();
    if (tokens == nullptr && x_in == nullptr)
        return fail(RWKV7_ERR_INVALID, "rwkv7_shift_mix: need x_in or tokens+emb");
    if (tokens != nullptr && (emb == nullptr || vocab <= 0))
        return fail(RWKV7_ERR_INVALID, "rwkv7_shift_mix: tokens need emb and vocab > 0");
    if ((ln0_w == nullptr) != (ln0_b == nullptr))
        return fail(RWKV7_ERR_INVALID, "rwkv7_shift_mix: ln0 weight and bias go together");
    if (!ln_w || !ln_b || !prev_pool || !row_slot || !row_last || !mix || !out)
        return fail(RWKV7_ERR_INVALID, "rwkv7_shift_mix: null pointer");
    if (bad_parts(add_parts, add, add_part_stride, M * C) || (add_parts > 0 && tokens != nullptr))
        return fail(RWKV7_ERR_INVALID, "rwkv7_shift_mix: bad partial sums (parts=%d stride=%lld; 1..%d planes of "
                    "M x C floats, 16-byte aligned, not with tokens)", add_parts, (long long)add_part_stride,
                    kMaxAddParts);
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_shift_mix<IO>((int)M, (int)C, x_in, add, add_parts, add_part_stride, tokens,
                                                emb, vocab, ln0_w, ln0_b,
                                                x_out, ln_w, ln_b, prev_pool, (int)pool_slots, row_slot,
                                                row_last, n_mix, mix, out, (hipStream_t)stream)));
    return launch_status(e, "shift_mix_kernel");
}

extern "C" int rwkv7_final_norm(int dtype, int64_t n, int64_t C, const float* x_in, const void* add,
                                int add_parts, int64_t add_part_stride, const int32_t* rows,
                                const float* ln_w, const float* ln_b, void* out, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_final_norm: bad dtype code %d", dtype);
    if (n < 0 || bad_c(C) || (C % 4) != 0 || n > kMaxInt) return fail(RWKV7_ERR_INVALID, "rwkv7_final_norm: bad sizes");
    if (n == 0) return ok();
    if (!x_in || !ln_w || !ln_b || !out) return fail(RWKV7_ERR_INVALID, "rwkv7_final_norm: null pointer");
    if (bad_parts(add_parts, add, add_part_stride, C))
        return fail(RWKV7_ERR_INVALID, "rwkv7_final_norm: bad partial sums (parts=%d stride=%lld)", add_parts,
                    (long long)add_part_stride);
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_final_norm<IO>((int)n, (int)C, x_in, add, add_parts, add_part_stride, rows,
                                                 ln_w, ln_b, out,
                                                 (hipStream_t)stream)));
    return launch_status(e, "final_norm_kernel");
}

extern "C" int rwkv7_activation(int dtype, int kind, int64_t n, void* x, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_activation: bad dtype code %d", dtype);
    if (kind < 0 || kind > 2) return fail(RWKV7_ERR_INVALID, "rwkv7_activation: kind must be 0, 1 or 2");
    if (n < 0 || n > ((int64_t)1 << 40)) return fail(RWKV7_ERR_INVALID, "rwkv7_activation: bad size");
    if (n == 0) return ok();
    if (!x) return fail(RWKV7_ERR_INVALID, "rwkv7_activation: null pointer");
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_activation<IO>(kind, n, x, (hipStream_t)stream)));
    return launch_status(e, "activation_kernel");
}

static bool params_ok(const float* const* p) {
    for (int i = 0; i < 8; ++i)
        if (p[i] == nullptr && i != 2) return false;  // v0 may be null on layer 0
    return true;
}

extern "C" int rwkv7_tmix_prep(int dtype, int64_t M, int64_t H, int layer0, const void* r, const void* k,
                               const void* v, const void* w_lora, const void* a_lora, const void* v_lora,
                               float* v_first, const float* const* params, void* const* wkv_ops,
                               void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_prep: bad dtype code %d", dtype);
    if (M < 0 || bad_h(H) || M > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_prep: bad sizes (H must be a positive multiple of 4)");
    if (M == 0) return ok();
    if (!params || !wkv_ops || !params_ok(params) || !r || !k || !v || !w_lora || !a_lora || !v_first)
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_prep: null pointer");
    if (!layer0 && (!v_lora || !params[2])) return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_prep: layer > 0 needs v_lora and v0");
    for (int i = 1; i < 6; ++i)  // wkv_ops[0] (the copy of r) may be null
        if (!wkv_ops[i]) return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_prep: null output");
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_tmix_prep<IO>((int)M, (int)H, layer0, r, k, v, w_lora, a_lora, v_lora,
                                                v_first, params, wkv_ops, (hipStream_t)stream)));
    return launch_status(e, "tmix_prep_kernel");
}

extern "C" int rwkv7_tmix_post(int dtype, int64_t M, int64_t H, const void* y, const void* r_op,
                               const void* k_op, const void* v_op, const void* g,
                               const float* const* params, void* out, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_post: bad dtype code %d", dtype);
    if (M < 0 || bad_h(H) || M > kMaxInt) return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_post: bad sizes");
    if (M == 0) return ok();
    if (!params || !params_ok(params) || !y || !r_op || !k_op || !v_op || !g || !out)
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_post: null pointer");
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_tmix_post<IO>((int)M, (int)H, y, r_op, k_op, v_op, g, params, out,
                                                (hipStream_t)stream)));
    return launch_status(e, "tmix_post_kernel");
}

extern "C" int rwkv7_tmix_decode(int dtype, int64_t M, int64_t H, int layer0, const void* r, const void* k,
                                 const void* v, const void* w_lora, const void* a_lora, const void* v_lora,
                                 const void* g, float* v_first, const float* const* params, float* state_pool,
                                 int64_t pool_slots, const int32_t* row_slot, void* out, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_decode: bad dtype code %d", dtype);
    if (M < 0 || bad_h(H) || pool_slots < 0 || M > kMaxInt || pool_slots > kMaxInt || M * H > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_decode: bad sizes (H must be a positive multiple of 4)");
    if (M == 0) return ok();
    if (!params || !params_ok(params) || !r || !k || !v || !w_lora || !a_lora || !g || !v_first ||
        !state_pool || !row_slot || !out)
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_decode: null pointer");
    if (((uintptr_t)state_pool & 15) != 0)
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_decode: state_pool must be aligned to 16 bytes");
    if (!layer0 && (!v_lora || !params[2]))
        return fail(RWKV7_ERR_INVALID, "rwkv7_tmix_decode: layer > 0 needs v_lora and v0");
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_tmix_decode<IO>((int)M, (int)H, layer0, r, k, v, w_lora, a_lora, v_lora, g,
                                                  v_first, params, state_pool, (int)pool_slots, row_slot,
                                                  out, (hipStream_t)stream)));
    return launch_status(e, "tmix_decode_kernel");
}

// ---------------------------------------------------------------------------
// Sampling (sampler.hip)
// ---------------------------------------------------------------------------

template <typename LT>
hipError_t launch_sample(int M, int V, const void* logits, int64_t ld, int rule, int max_valid_id,
                         const float* temperature, const float* top_p, const int32_t* top_k,
                         const int32_t* bias_off, const int32_t* bias_ids, const float* bias_val,
                         const uint8_t* active, uint64_t seed, const int64_t* rng_key,
                         const int32_t* rng_ctr, int64_t* out_tok, float* out_logp, hipStream_t st);
hipError_t launch_rep_penalty(int M, int V, float* logits, int64_t ld, float penalty, const int32_t* hist,
                              const int64_t* hist_start, const int32_t* hist_len, const int32_t* hist2,
                              const int64_t* hist2_start, const int32_t* hist2_len, const uint8_t* active,
                              hipStream_t st);
int sampler_max_vocab();

extern "C" int rwkv7_sample(int dtype, int64_t M, int64_t V, const void* logits, int64_t ld, int rule,
                            int64_t max_valid_id, const float* temperature, const float* top_p,
                            const int32_t* top_k, const int32_t* bias_off, const int32_t* bias_ids,
                            const float* bias_val, const uint8_t* active, uint64_t seed,
                            const int64_t* rng_key, const int32_t* rng_ctr, int64_t* out_tok,
                            float* out_logp, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_sample: bad dtype code %d", dtype);
    if (M < 0 || M > kMaxInt || V <= 0 || V > sampler_max_vocab() || ld < V)
        return fail(RWKV7_ERR_INVALID, "rwkv7_sample: bad sizes M=%lld V=%lld ld=%lld (V <= %d)", (long long)M,
                    (long long)V, (long long)ld, sampler_max_vocab());
    if (rule < 0 || rule > 2)
        return fail(RWKV7_ERR_INVALID, "rwkv7_sample: rule must be 0 (batch), 1 (single) or 2 (generate)");
    if (M == 0) return ok();
    if (!logits || !temperature || !top_p || !top_k || !rng_key || !rng_ctr || !out_tok || !out_logp)
        return fail(RWKV7_ERR_INVALID, "rwkv7_sample: null pointer");
    if (bias_off != nullptr && (bias_ids == nullptr || bias_val == nullptr))
        return fail(RWKV7_ERR_INVALID, "rwkv7_sample: bias_off needs bias_ids and bias_val");
    const int mv = max_valid_id < 0 ? (int)(V - 1) : (int)(max_valid_id < V ? max_valid_id : V - 1);
    hipError_t e;
    switch (dtype) {
        case RWKV7_DTYPE_F32:
            e = launch_sample<float>((int)M, (int)V, logits, ld, rule, mv, temperature, top_p, top_k, bias_off,
                                     bias_ids, bias_val, active, seed, rng_key, rng_ctr, out_tok, out_logp,
                                     (hipStream_t)stream);
            break;
        case RWKV7_DTYPE_F16:
            e = launch_sample<f16_t>((int)M, (int)V, logits, ld, rule, mv, temperature, top_p, top_k, bias_off,
                                     bias_ids, bias_val, active, seed, rng_key, rng_ctr, out_tok, out_logp,
                                     (hipStream_t)stream);
            break;
        default:
            e = launch_sample<bf16_t>((int)M, (int)V, logits, ld, rule, mv, temperature, top_p, top_k, bias_off,
                                      bias_ids, bias_val, active, seed, rng_key, rng_ctr, out_tok, out_logp,
                                      (hipStream_t)stream);
            break;
    }
    return launch_status(e, "sample_kernel");
}

extern "C" int rwkv7_repetition_penalty(int64_t M, int64_t V, float* logits, int64_t ld, float penalty,
                                        const int32_t* hist, const int64_t* hist_start, const int32_t* hist_len,
                                        const int32_t* hist2, const int64_t* hist2_start,
                                        const int32_t* hist2_len, const uint8_t* active, void* stream) {
    if (M < 0 || M > kMaxInt || V <= 0 || V > kMaxInt || ld < V)
        return fail(RWKV7_ERR_INVALID, "rwkv7_repetition_penalty: bad sizes");
    if (penalty == 1.0f || penalty <= 0.0f || M == 0) return ok();  // no-op, as the reference
    if (!logits || !hist || !hist_start || !hist_len)
        return fail(RWKV7_ERR_INVALID, "rwkv7_repetition_penalty: null pointer");
    if (hist2 != nullptr && (hist2_start == nullptr || hist2_len == nullptr))
        return fail(RWKV7_ERR_INVALID, "rwkv7_repetition_penalty: hist2 needs hist2_start and hist2_len");
    return launch_status(launch_rep_penalty((int)M, (int)V, logits, ld, penalty, hist, hist_start, hist_len, hist2,
                                            hist2_start, hist2_len, active, (hipStream_t)stream),
                         "rep_penalty_kernel");
}

// ---------------------------------------------------------------------------
// Slot table (slots.hip)
// ---------------------------------------------------------------------------

hipError_t launch_rollout_first(int n, const int32_t* seq_idx, int n_seq, int maxlen, const int64_t* tok,
                                const float* logp, const int32_t* seq_max_new, int32_t* seq_ngen, uint8_t* seq_done,
                                int32_t* out_tok, float* out_logp, int32_t* out_step, int64_t eos,
                                int first_can_finish, int32_t* counters, hipStream_t st);
hipError_t launch_rollout_commit(int S, int n, int maxlen, int have_sample, const int64_t* tok, const float* logp,
                                 int32_t* slot_seq, int32_t* row_slot, int32_t* slot_row, int64_t* tok_in,
                                 const int32_t* seq_prompt,
                                 const int32_t* seq_max_new, int32_t* seq_ngen, uint8_t* seq_done,
                                 int32_t* out_tok, float* out_logp, int32_t* out_step, int64_t eos,
                                 int32_t* counters, int32_t* admit_slot, int32_t* admit_src, hipStream_t st);
hipError_t launch_rollout_prepare(int S, int maxlen, const int32_t* row_slot, const int32_t* slot_seq,
                                  const int64_t* seq_key, const int32_t* seq_ngen,
                                  const int32_t* seq_prompt, const int64_t* prompt_start,
                                  const int32_t* prompt_len, uint8_t* active, int64_t* rng_key,
                                  int32_t* rng_ctr, int64_t* hist_start, int32_t* hist_len,
                                  int64_t* hist2_start, int32_t* hist2_len, const float* seq_temp,
                                  const float* seq_top_p, const int32_t* seq_top_k, float* temp, float* top_p,
                                  int32_t* top_k, hipStream_t st);
hipError_t launch_admit_copy(const int32_t* counters, const int32_t* admit_slot, const int32_t* admit_src, int L,
                             int S, int U, int64_t kv_elems, int64_t C, const float* src_kv, const float* src_ax,
                             const float* src_fx, float* dst_kv, float* dst_ax, float* dst_fx, hipStream_t st);

extern "C" int rwkv7_rollout_first(int64_t n, int64_t maxlen, const int64_t* tok, const float* logp,
                                   const int32_t* seq_max_new, int32_t* seq_ngen, uint8_t* seq_done,
                                   int32_t* out_tok, float* out_logp, int32_t* out_step, int64_t eos,
                                   int first_can_finish, int32_t* counters, void* stream) {
    if (n < 0 || n > kMaxInt || maxlen < 1 || maxlen > kMaxInt || n * maxlen > ((int64_t)1 << 40))
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_first: bad sizes");
    if (n == 0) return ok();
    if (!tok || !logp || !seq_max_new || !seq_ngen || !seq_done || !out_tok || !out_logp || !counters)
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_first: null pointer");
    return launch_status(launch_rollout_first((int)n, nullptr, (int)n, (int)maxlen, tok, logp, seq_max_new, seq_ngen,
                                              seq_done, out_tok, out_logp, out_step, eos, first_can_finish, counters,
                                              (hipStream_t)stream),
                         "rollout_first_kernel");
}

extern "C" int rwkv7_rollout_activate(int64_t m, const int32_t* seq_idx, int64_t n, int64_t maxlen,
                                      const int64_t* tok, const float* logp, const int32_t* seq_max_new,
                                      int32_t* seq_ngen, uint8_t* seq_done, int32_t* out_tok, float* out_logp,
                                      int32_t* out_step, int64_t eos, int first_can_finish, int32_t* counters,
                                      void* stream) {
    if (m < 0 || m > kMaxInt || n < 0 || n > kMaxInt || maxlen < 1 || maxlen > kMaxInt ||
        n * maxlen > ((int64_t)1 << 40))
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_activate: bad sizes");
    if (m == 0) return ok();
    if (!seq_idx || !tok || !logp || !seq_max_new || !seq_ngen || !seq_done || !out_tok || !out_logp || !counters)
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_activate: null pointer");
    return launch_status(launch_rollout_first((int)m, seq_idx, (int)n, (int)maxlen, tok, logp, seq_max_new, seq_ngen,
                                              seq_done, out_tok, out_logp, out_step, eos, first_can_finish, counters,
                                              (hipStream_t)stream),
                         "rollout_first_kernel");
}

extern "C" int rwkv7_rollout_commit(int64_t S, int64_t n, int64_t maxlen, int have_sample, const int64_t* tok,
                                    const float* logp, int32_t* slot_seq, int32_t* row_slot, int32_t* slot_row,
                                    int64_t* tok_in,
                                    const int32_t* seq_prompt, const int32_t* seq_max_new, int32_t* seq_ngen,
                                    uint8_t* seq_done, int32_t* out_tok, float* out_logp, int32_t* out_step,
                                    int64_t eos, int32_t* counters, int32_t* admit_slot, int32_t* admit_src,
                                    void* stream) {
    if (S < 1 || S > 1024 || n < 0 || n > kMaxInt || maxlen < 1 || maxlen > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_commit: bad sizes (1 <= S <= 1024)");
    if (have_sample && (!tok || !logp)) return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_commit: null sample");
    if (!slot_seq || !row_slot || !tok_in || !seq_prompt || !seq_max_new || !seq_ngen || !seq_done || !out_tok ||
        !out_logp || !counters || !admit_slot || !admit_src)
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_commit: null pointer");
    return launch_status(launch_rollout_commit((int)S, (int)n, (int)maxlen, have_sample, tok, logp, slot_seq, row_slot,
                                               slot_row, tok_in, seq_prompt, seq_max_new, seq_ngen, seq_done, out_tok,
                                               out_logp, out_step, eos, counters, admit_slot, admit_src,
                                               (hipStream_t)stream),
                         "rollout_commit_kernel");
}

extern "C" int rwkv7_rollout_prepare(int64_t S, int64_t maxlen, const int32_t* row_slot, const int32_t* slot_seq,
                                     const int64_t* seq_key, const int32_t* seq_ngen,
                                     const int32_t* seq_prompt, const int64_t* prompt_start,
                                     const int32_t* prompt_len, uint8_t* active, int64_t* rng_key,
                                     int32_t* rng_ctr, int64_t* hist_start, int32_t* hist_len,
                                     int64_t* hist2_start, int32_t* hist2_len, const float* seq_temp,
                                     const float* seq_top_p, const int32_t* seq_top_k, float* temp,
                                     float* top_p, int32_t* top_k, void* stream) {
    if (S < 1 || S > kMaxInt || maxlen < 1 || maxlen > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_prepare: bad sizes");
    if (!slot_seq || !seq_ngen || !active || !rng_key || !rng_ctr)
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_prepare: null pointer");
    if (hist_start && (!seq_prompt || !prompt_start || !prompt_len || !hist_len || !hist2_start || !hist2_len))
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_prepare: history outputs need the prompt table");
    if (seq_temp && (!seq_top_p || !seq_top_k || !temp || !top_p || !top_k))
        return fail(RWKV7_ERR_INVALID, "rwkv7_rollout_prepare: per-sequence parameters come as a set");
    return launch_status(launch_rollout_prepare((int)S, (int)maxlen, row_slot, slot_seq, seq_key, seq_ngen, seq_prompt,
                                                prompt_start,
                                                prompt_len, active, rng_key, rng_ctr, hist_start, hist_len,
                                                hist2_start, hist2_len, seq_temp, seq_top_p, seq_top_k, temp,
                                                top_p, top_k, (hipStream_t)stream),
                         "rollout_prepare_kernel");
}

extern "C" int rwkv7_admit_copy(const int32_t* counters, const int32_t* admit_slot, const int32_t* admit_src,
                                int64_t L, int64_t S, int64_t U, int64_t kv_elems, int64_t C, const float* src_kv,
                                const float* src_ax, const float* src_fx, float* dst_kv, float* dst_ax,
                                float* dst_fx, void* stream) {
    if (L < 1 || S < 1 || U < 1 || kv_elems < 4 || (kv_elems % 4) || C < 4 || (C % 4) || S > kMaxInt || U > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_admit_copy: bad sizes");
    if (!counters || !admit_slot || !admit_src || !src_kv || !src_ax || !src_fx || !dst_kv || !dst_ax || !dst_fx)
        return fail(RWKV7_ERR_INVALID, "rwkv7_admit_copy: null pointer");
    return launch_status(launch_admit_copy(counters, admit_slot, admit_src, (int)L, (int)S, (int)U, kv_elems, C,
                                           src_kv, src_ax, src_fx, dst_kv, dst_ax, dst_fx, (hipStream_t)stream),
                         "admit_copy_kernel");
}

// ---------------------------------------------------------------------------
// Training operator (wkv7_train.hip)
// ---------------------------------------------------------------------------

int64_t wkv7_train_ckpt_floats(int B, int T, int H);
template <typename IO>
hipError_t launch_wkv7_train_fwd(int B, int T, int H, const void* r, const void* w, const void* k, const void* v,
                                 const void* a, const void* b, void* y, const float* s0, float* s_out, float* ckpt,
                                 float* sa, hipStream_t st);
template <typename IO>
hipError_t launch_wkv7_train_bwd(int B, int T, int H, const void* r, const void* w, const void* k, const void* v,
                                 const void* a, const void* b, const void* dy, const float* ckpt, const float* sa,
                                 const float* ds_in, void* dr, void* dw, void* dk, void* dv, void* da, void* db,
                                 float* ds0, hipStream_t st);
template <typename IO>
hipError_t launch_wkv7_chunk_train(int B, int T, int H, const void* r, const void* w, const void* k, const void* v,
                                   const void* a, const void* b, void* y, const float* s0, float* s_out, float* ckpt,
                                   float* sa, hipStream_t stream);

namespace {
int train_sizes(const char* fn, int64_t B, int64_t T, int64_t H) {
    if (B < 0 || T < 0 || H <= 0)
        return fail(RWKV7_ERR_INVALID, "%s: bad sizes B=%lld T=%lld H=%lld", fn, (long long)B, (long long)T,
                    (long long)H);
    if (B * H > kMaxInt || T > kMaxInt || B * T * H * RWKV7_HEAD > ((int64_t)1 << 40))
        return fail(RWKV7_ERR_INVALID, "%s: problem too large", fn);
    return RWKV7_OK;
}
bool f32_misaligned(const float* p) { return (((uintptr_t)p) & 15) != 0; }
}  // namespace

extern "C" int64_t rwkv7_wkv_train_ckpt_floats(int64_t B, int64_t T, int64_t H) {
    if (train_sizes("rwkv7_wkv_train_ckpt_floats", B, T, H) != RWKV7_OK) return -1;
    ok();
    return wkv7_train_ckpt_floats((int)B, (int)T, (int)H);
}

extern "C" int rwkv7_wkv_train_forward(int dtype, int64_t B, int64_t T, int64_t H, const void* r, const void* w,
                                       const void* k, const void* v, const void* a, const void* b, void* y,
                                       const float* s0, float* s_out, float* ckpt, float* sa, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_forward: bad dtype code %d", dtype);
    if (train_sizes("rwkv7_wkv_train_forward", B, T, H) != RWKV7_OK) return RWKV7_ERR_INVALID;
    if (B == 0 || T == 0) return ok();
    if (any_null(r, w, k, v, a, b, y, ckpt) || !sa)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_forward: null pointer");
    if (f32_misaligned(ckpt) || f32_misaligned(s0) || f32_misaligned(s_out))
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_forward: checkpoints and states must be 16-byte aligned");
    hipError_t e;
    // 16-bit inputs aligned to 4 elements run the chunked kernel (32-token matrix
    // form on the matrix cores); float32 inputs keep the token-serial kernel
    if (dtype != RWKV7_DTYPE_F32 && B * T <= kMaxInt && !misaligned(dtype, nullptr, r, w, k, v, a, b)) {
        if (dtype == RWKV7_DTYPE_F16)
            e = launch_wkv7_chunk_train<f16_t>((int)B, (int)T, (int)H, r, w, k, v, a, b, y, s0, s_out, ckpt, sa,
                                               (hipStream_t)stream);
        else
            e = launch_wkv7_chunk_train<bf16_t>((int)B, (int)T, (int)H, r, w, k, v, a, b, y, s0, s_out, ckpt, sa,
                                                (hipStream_t)stream);
        return launch_status(e, "wkv7_chunk2_kernel (training)");
    }
    RWKV7_DISPATCH(dtype, (launch_wkv7_train_fwd<IO>((int)B, (int)T, (int)H, r, w, k, v, a, b, y, s0, s_out, ckpt,
                                                     sa, (hipStream_t)stream)));
    return launch_status(e, "wkv7_train_fwd_kernel");
}

extern "C" int rwkv7_wkv_train_backward(int dtype, int64_t B, int64_t T, int64_t H, const void* r, const void* w,
                                        const void* k, const void* v, const void* a, const void* b, const void* dy,
                                        const float* ckpt, const float* sa, const float* ds_in, void* dr, void* dw,
                                        void* dk, void* dv, void* da, void* db, float* ds0, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_backward: bad dtype code %d", dtype);
    if (train_sizes("rwkv7_wkv_train_backward", B, T, H) != RWKV7_OK) return RWKV7_ERR_INVALID;
    if (B == 0) return ok();
    if (T == 0) {
        if (ds0 == nullptr) return ok();
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_backward: T = 0 with an initial-state gradient "
                    "(copy ds_in instead)");
    }
    if (any_null(r, w, k, v, a, b, dy, ckpt) || !sa || any_null(dr, dw, dk, dv, da, db, sa, ckpt))
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_backward: null pointer");
    if (f32_misaligned(ckpt) || f32_misaligned(ds0))
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_train_backward: checkpoints and ds0 must be 16-byte aligned");
    hipError_t e;
    RWKV7_DISPATCH(dtype, (launch_wkv7_train_bwd<IO>((int)B, (int)T, (int)H, r, w, k, v, a, b, dy, ckpt, sa, ds_in,
                                                     dr, dw, dk, dv, da, db, ds0, (hipStream_t)stream)));
    return launch_status(e, "wkv7_train_bwd_kernel");
}

// ---------------------------------------------------------------------------
// Grouped decode GEMM (gemm_decode.hip)
// ---------------------------------------------------------------------------

hipError_t launch_gemm_decode(int M, int count, const void* const* A, const void* const* B, void* const* C,
                              const int64_t* lda, const int64_t* ldc, const int* N, const int* K,
                              const int* epi, float* ws, hipStream_t st);
int gemm_decode_max_problems();
int64_t gemm_decode_workspace(int M, int count, const int* N, const int* K);
int64_t gemm_packed_elems(int N, int K);
hipError_t launch_gemm_pack(const void* B, int64_t ldb, int N, int K, void* out, hipStream_t st);
int gemm_decode_partial_splits(int M, int N, int K);
hipError_t launch_gemm_decode_partials(int M, const void* A, const void* B, int64_t lda, int N, int K, float* ws,
                                       hipStream_t st);
namespace {
int check_gemm_problems(const char* fn, int64_t M, int count, const int* N, const int* K) {
    if (count < 1 || count > gemm_decode_max_problems())
        return fail(RWKV7_ERR_INVALID, "%s: 1 <= count <= %d", fn, gemm_decode_max_problems());
    if (M < 0 || M > (1 << 20)) return fail(RWKV7_ERR_INVALID, "%s: bad M=%lld", fn, (long long)M);
    if (!N || !K) return fail(RWKV7_ERR_INVALID, "%s: null array", fn);
    for (int i = 0; i < count; ++i)
        if (N[i] <= 0 || K[i] <= 0 || (K[i] % 8) != 0)
            return fail(RWKV7_ERR_INVALID, "%s: problem %d: N > 0, K > 0 and K %% 8 == 0 required", fn, i);
    return RWKV7_OK;
}
}  // namespace

extern "C" int64_t rwkv7_gemm_decode_workspace(int64_t M, int count, const int* N, const int* K) {
    if (check_gemm_problems("rwkv7_gemm_decode_workspace", M, count, N, K) != RWKV7_OK) return -1;
    ok();
    return gemm_decode_workspace((int)(M > 0 ? M : 1), count, N, K);
}

namespace {
// Argument checks shared by rwkv7_gemm_decode and rwkv7_gemm_decode_noalloc;
// *need_ws receives the split-K floats the problem set needs.
int check_gemm_decode(const char* fn, int64_t M, int count, const void* const* A, const void* const* B,
                      void* const* C, const int64_t* lda, const int64_t* ldc, const int* N, const int* K,
                      const int* epi, int64_t* need_ws) {
    if (check_gemm_problems(fn, M, count, N, K) != RWKV7_OK) return RWKV7_ERR_INVALID;
    *need_ws = 0;
    if (M == 0) return RWKV7_OK;
    if (!A || !B || !C || !lda || !ldc || !epi) return fail(RWKV7_ERR_INVALID, "%s: null array", fn);
    int64_t blocks = 0;
    for (int i = 0; i < count; ++i) {
        if (!A[i] || !B[i] || !C[i]) return fail(RWKV7_ERR_INVALID, "%s: null pointer in problem %d", fn, i);
        if (lda[i] < K[i] || ldc[i] < N[i] || (lda[i] % 8) != 0)
            return fail(RWKV7_ERR_INVALID, "%s: problem %d: lda >= K and %% 8 == 0, ldc >= N required", fn, i);
        if ((((uintptr_t)A[i]) | ((uintptr_t)B[i])) & 15)
            return fail(RWKV7_ERR_INVALID, "%s: problem %d: A and packed B must be 16-byte aligned", fn, i);
        if (epi[i] < 0 || epi[i] > 3) return fail(RWKV7_ERR_INVALID, "%s: problem %d: epi in 0..3", fn, i);
        blocks += ((M + 31) / 32) * (int64_t)((N[i] + 63) / 64 + 7) * 8;
    }
    if (blocks > kMaxInt) return fail(RWKV7_ERR_INVALID, "%s: too many tiles", fn);
    *need_ws = gemm_decode_workspace((int)M, count, N, K);
    return RWKV7_OK;
}
}  // namespace

extern "C" int rwkv7_gemm_decode(int64_t M, int count, const void* const* A, const void* const* B, void* const* C,
                                 const int64_t* lda, const int64_t* ldc, const int* N, const int* K, const int* epi,
                                 float* workspace, int64_t workspace_floats, void* stream) {
    int64_t need_ws = 0;
    const int rc = check_gemm_decode("rwkv7_gemm_decode", M, count, A, B, C, lda, ldc, N, K, epi, &need_ws);
    if (rc != RWKV7_OK) return rc;
    if (M == 0) return ok();
    if (need_ws > 0 && (workspace == nullptr || workspace_floats < need_ws))
        return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode: needs a workspace of %lld floats (have %lld)",
                    (long long)need_ws, (long long)workspace_floats);
    return launch_status(launch_gemm_decode((int)M, count, A, B, C, lda, ldc, N, K, epi, workspace,
                                            (hipStream_t)stream),
                         "gemm_decode_kernel");
}

hipError_t gemm_scratch(float** out);

extern "C" int rwkv7_gemm_decode_noalloc(int64_t M, int count, const void* const* A, const void* const* B,
                                         void* const* C, const int64_t* lda, const int64_t* ldc, const int* N,
                                         const int* K, const int* epi, void* stream) {
    int64_t need_ws = 0;
    const int rc = check_gemm_decode("rwkv7_gemm_decode_noalloc", M, count, A, B, C, lda, ldc, N, K, epi, &need_ws);
    if (rc != RWKV7_OK) return rc;
    if (M == 0) return ok();
    if (need_ws > RWKV7_GEMM_SCRATCH_FLOATS)
        return fail(RWKV7_ERR_INVALID,
                    "rwkv7_gemm_decode_noalloc: this problem set needs %lld floats of split-K scratch, more than "
                    "the %lld of the library's static scratch; use rwkv7_gemm_decode with a workspace",
                    (long long)need_ws, (long long)RWKV7_GEMM_SCRATCH_FLOATS);
    float* ws = nullptr;
    if (need_ws > 0) {
        const hipError_t e = gemm_scratch(&ws);
        if (e != hipSuccess)
            return fail(RWKV7_ERR_LAUNCH, "rwkv7_gemm_decode_noalloc: scratch address: %s", hipGetErrorString(e));
    }
    return launch_status(launch_gemm_decode((int)M, count, A, B, C, lda, ldc, N, K, epi, ws, (hipStream_t)stream),
                         "gemm_decode_kernel");
}

extern "C" int rwkv7_gemm_decode_partial_count(int64_t M, int N, int K) {
    if (check_gemm_problems("rwkv7_gemm_decode_partial_count", M, 1, &N, &K) != RWKV7_OK) return -1;
    ok();
    return gemm_decode_partial_splits((int)(M > 0 ? M : 1), N, K);
}

extern "C" int rwkv7_gemm_decode_partials(int64_t M, const void* A, const void* B, int64_t lda, int N, int K,
                                          float* workspace, int64_t workspace_floats, int32_t* parts,
                                          void* stream) {
    if (check_gemm_problems("rwkv7_gemm_decode_partials", M, 1, &N, &K) != RWKV7_OK) return RWKV7_ERR_INVALID;
    if (!parts) return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode_partials: null parts");
    const int np = gemm_decode_partial_splits((int)(M > 0 ? M : 1), N, K);
    *parts = np;
    if (M == 0) return ok();
    if (!A || !B) return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode_partials: null pointer");
    if (lda < K || (lda % 8) != 0)
        return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode_partials: lda >= K and lda %% 8 == 0 required");
    if ((((uintptr_t)A) | ((uintptr_t)B) | ((uintptr_t)workspace)) & 15)
        return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode_partials: A, packed B and the workspace must be 16-byte "
                    "aligned");
    if (((M + 31) / 32) * (int64_t)((N + 63) / 64 + 7) * 8 * np > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode_partials: too many tiles");
    const int64_t need_ws = (int64_t)np * M * N;
    if (workspace == nullptr || workspace_floats < need_ws)
        return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_decode_partials: needs a workspace of %lld floats (have %lld)",
                    (long long)need_ws, (long long)workspace_floats);
    return launch_status(launch_gemm_decode_partials((int)M, A, B, lda, N, K, workspace, (hipStream_t)stream),
                         "gemm_decode_kernel");
}

extern "C" int64_t rwkv7_gemm_packed_elems(int N, int K) {
    if (N <= 0 || K <= 0 || (K % 8) != 0 || N > (1 << 24) || K > (1 << 24)) {
        fail(RWKV7_ERR_INVALID, "rwkv7_gemm_packed_elems: N > 0, K > 0, K %% 8 == 0 required");
        return -1;
    }
    ok();
    return gemm_packed_elems(N, K);
}

extern "C" int rwkv7_gemm_pack(const void* B, int64_t ldb, int N, int K, void* out, void* stream) {
    if (rwkv7_gemm_packed_elems(N, K) < 0) return RWKV7_ERR_INVALID;
    if (!B || !out) return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_pack: null pointer");
    if (ldb < K || (ldb % 8) != 0 || ((((uintptr_t)B) | ((uintptr_t)out)) & 15))
        return fail(RWKV7_ERR_INVALID, "rwkv7_gemm_pack: ldb >= K, ldb %% 8 == 0 and 16-byte aligned buffers required");
    return launch_status(launch_gemm_pack(B, ldb, N, K, out, (hipStream_t)stream), "gemm_pack_kernel");
}

// ---------------------------------------------------------------------------
// LM head for decode rows (head_gemm.hip)
// ---------------------------------------------------------------------------

int head_min_k();
int head_row_tile(int M);
int64_t head_packed_elems(int V, int K);
hipError_t launch_head_logits(int M, int V, int K, const void* A, int64_t lda, const void* Bp, void* C, int64_t ldc,
                              hipStream_t st);
hipError_t launch_head_pack(const void* W, int64_t ldw, int V, int K, void* out, hipStream_t st);

extern "C" int64_t rwkv7_head_packed_elems(int V, int K) {
    if (V <= 0 || K <= 0 || (K % 64) != 0 || V > (1 << 24) || K > (1 << 16)) {
        fail(RWKV7_ERR_INVALID, "rwkv7_head_packed_elems: 0 < V <= 2^24, 0 < K <= 65536, K %% 64 == 0 required "
             "(V=%d K=%d)", V, K);
        return -1;
    }
    ok();
    return head_packed_elems(V, K);
}

extern "C" int rwkv7_head_pack(const void* W, int64_t ldw, int V, int K, void* out, void* stream) {
    if (rwkv7_head_packed_elems(V, K) < 0) return RWKV7_ERR_INVALID;
    if (!W || !out) return fail(RWKV7_ERR_INVALID, "rwkv7_head_pack: null pointer");
    if (ldw < K || (ldw % 8) != 0 || ((((uintptr_t)W) | ((uintptr_t)out)) & 15))
        return fail(RWKV7_ERR_INVALID, "rwkv7_head_pack: ldw >= K, ldw %% 8 == 0 and 16-byte aligned buffers required");
    return launch_status(launch_head_pack(W, ldw, V, K, out, (hipStream_t)stream), "head_pack_kernel");
}

extern "C" int rwkv7_head_logits(int64_t M, int V, int K, const void* A, int64_t lda, const void* W_packed,
                                 void* logits, int64_t ldc, void* stream) {
    if (M < 0 || M > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_head_logits: 0 <= M <= 2^31 - 1 required (M=%lld)", (long long)M);
    if (V <= 0 || (V % 256) != 0 || V > (1 << 24) || (K % 64) != 0 || K < head_min_k() || K > (1 << 16))
        return fail(RWKV7_ERR_INVALID, "rwkv7_head_logits: V %% 256 == 0, K %% 64 == 0 and %d <= K <= 65536 required "
                    "(V=%d K=%d)", head_min_k(), V, K);
    if (M == 0) return ok();
    if (!A || !W_packed || !logits) return fail(RWKV7_ERR_INVALID, "rwkv7_head_logits: null pointer");
    if (lda < K || (lda % 8) != 0 || ldc < V || (ldc % 8) != 0)
        return fail(RWKV7_ERR_INVALID, "rwkv7_head_logits: lda >= K, ldc >= V, both multiples of 8 required");
    if ((((uintptr_t)A) | ((uintptr_t)W_packed) | ((uintptr_t)logits)) & 15)
        return fail(RWKV7_ERR_INVALID, "rwkv7_head_logits: A, the packed weight and the logits must be 16-byte "
                    "aligned");
    const int bm = head_row_tile((int)M);
    if ((M + bm - 1) / bm > 65535) return fail(RWKV7_ERR_INVALID, "rwkv7_head_logits: too many rows");
    return launch_status(launch_head_logits((int)M, V, K, A, lda, W_packed, logits, ldc, (hipStream_t)stream),
                         "head_logits_kernel");
}

// ---------------------------------------------------------------------------
// Selective log-softmax (logprob.hip)
// ---------------------------------------------------------------------------

template <typename LT>
hipError_t launch_selective_logsoftmax(int R, int V, const void* logits, int64_t ld, const int64_t* index, void* out,
                                       hipStream_t st);

extern "C" int rwkv7_selective_log_softmax(int dtype, int64_t R, int64_t V, const void* logits, int64_t ld,
                                           const int64_t* index, void* out, void* stream) {
    if (!dtype_ok(dtype)) return fail(RWKV7_ERR_INVALID, "rwkv7_selective_log_softmax: bad dtype %d", dtype);
    if (R < 0 || R > kMaxInt || V < 1 || V > kMaxInt || ld < V)
        return fail(RWKV7_ERR_INVALID, "rwkv7_selective_log_softmax: need 0 <= R, 1 <= V <= ld (R=%lld V=%lld ld=%lld)",
                    (long long)R, (long long)V, (long long)ld);
    if (R == 0) return ok();
    if (!logits || !index || !out) return fail(RWKV7_ERR_INVALID, "rwkv7_selective_log_softmax: null pointer");
    hipError_t e;
    switch (dtype) {
        case RWKV7_DTYPE_F32:
            e = launch_selective_logsoftmax<float>((int)R, (int)V, logits, ld, index, out, (hipStream_t)stream);
            break;
        case RWKV7_DTYPE_F16:
            e = launch_selective_logsoftmax<f16_t>((int)R, (int)V, logits, ld, index, out, (hipStream_t)stream);
            break;
        default:
            e = launch_selective_logsoftmax<bf16_t>((int)R, (int)V, logits, ld, index, out, (hipStream_t)stream);
            break;
    }
    return launch_status(e, "selective_logsoftmax_kernel");
}
