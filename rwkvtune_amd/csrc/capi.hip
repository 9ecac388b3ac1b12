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

bool any_null(const void* p0, const void* p1, const void* p2, const void* p3, const void* p4,
              const void* p5, const void* p6, const void* p7) {
    return !p0 || !p1 || !p2 || !p3 || !p4 || !p5 || !p6 || !p7;
}

}  // namespace

extern "C" int rwkv7_abi_version(void) { return 1; }

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
    if (B * T > kMaxInt || B * H > kMaxInt || B * T * C > (int64_t)1 << 40)
        return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: problem too large");
    if (any_null(state, r, w, k, v, a, b, y)) return fail(RWKV7_ERR_INVALID, "rwkv7s_forward: null pointer");
    hipStream_t st = (hipStream_t)stream;
    return seq_dispatch(dtype, (int)B, (int)H, (int)T, nullptr, nullptr, (int)B, (int)(B * T), state,
                        r, w, k, v, a, b, y, st);
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
    if (B * H > kMaxInt || pool_slots > kMaxInt) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: too large");
    if (any_null(state_pool, r, w, k, v, a, b, y)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_decode: null pointer");
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
    if (chunk_len != 0 && chunk_len != 16 && chunk_len != 32 && chunk_len != 64)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: chunk_len must be 0, 16, 32 or 64 (got %d)", chunk_len);
    if (nseq == 0 || total_tokens == 0) return ok();
    if (cu_seqlens == nullptr) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: cu_seqlens is required");
    if (slot_idx == nullptr && pool_slots < nseq)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: identity slots need pool_slots >= nseq");
    if (nseq * H > kMaxInt || total_tokens > kMaxInt || pool_slots > kMaxInt)
        return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: too large");
    if (any_null(state_pool, r, w, k, v, a, b, y)) return fail(RWKV7_ERR_INVALID, "rwkv7_wkv_prefill: null pointer");
    return seq_dispatch(dtype, (int)nseq, (int)H, 0, cu_seqlens, slot_idx, (int)pool_slots, (int)total_tokens,
                        state_pool, r, w, k, v, a, b, y, (hipStream_t)stream);
}
