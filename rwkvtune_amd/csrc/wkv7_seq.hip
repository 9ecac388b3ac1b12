// WKV7 token-serial kernel for gfx950: single-token decode (T = 1) and short
// prefills.  Semantics follow the reference kernel
// rwkvtune/models/rwkv7/operators/cuda/wkv7s.cu:5-54 (per token: decay
// exp(-exp(w_raw)), sa = S a, S <- S diag(w) + v k^T + sa b^T, y = S r), with
// these design differences:
//   * rows of the state do not interact in a step, so a (sequence, head) unit
//     is split into four quarters of 16 rows, one single-wave block each
//     (block 4 unit + q), streaming its contiguous 4 KB of the unit's 16 KB
//     state with coalesced, non-temporal 128-bit accesses: lane l = 16g + c holds
//     S[16q + 4m + g][4c..4c+3] for m = 0..3.  Quarter-unit waves keep more
//     state loads in flight per CU than whole-unit ones (in-place read-write
//     streaming measured on MI355X: 77% of HBM peak for 4 KB per wave, 74% for
//     16 KB; cfg2 decode 73.6% -> 74.9%);
//   * row reductions (S a and S r) are DPP butterflies inside 16-lane rows;
//   * the state is addressed through an optional slot table
//     (slot_idx[s] = pool slot of sequence s, negative = inactive, skipped),
//     so decode runs on a resident [slots, H, N, N] pool without gather/scatter;
//   * ragged batches: token range of sequence s is [cu[s], cu[s+1]) of a packed
//     [total, C] layout (or [s*T, s*T+T) for the uniform [B, T, C] layout).
#include "common.hpp"

namespace {

template <typename IO>
__global__ __launch_bounds__(64) void wkv7_seq_kernel(
    const int H, const int T_uniform, const int32_t* __restrict__ cu_seqlens,
    const int32_t* __restrict__ slot_idx, const int pool_slots, const int total_tokens,
    float* __restrict__ state, const IO* __restrict__ r, const IO* __restrict__ w,
    const IO* __restrict__ k, const IO* __restrict__ v, const IO* __restrict__ a,
    const IO* __restrict__ b, IO* __restrict__ y)
{
    typedef io_traits<IO> tr;
    const int unit = blockIdx.x >> 2;
    const int q = blockIdx.x & 3;
    const int s = unit / H;
    const int h = unit - s * H;
    const int l = threadIdx.x;
    const int g = l >> 4;
    const int c = l & 15;

    int t0, t1;
    if (cu_seqlens != nullptr) {
        t0 = cu_seqlens[s];
        t1 = cu_seqlens[s + 1];
        if (t0 < 0 || t1 < t0 || t1 > total_tokens) return;  // malformed row: leave untouched
    } else {
        t0 = s * T_uniform;
        t1 = t0 + T_uniform;
    }
    if (t1 == t0) return;
    const int slot = slot_idx != nullptr ? slot_idx[s] : s;
    if (slot < 0 || slot >= pool_slots) return;  // inactive slot

    const int C = H * RWKV7_HEAD;
    f32x4* sp = reinterpret_cast<f32x4*>(state + ((size_t)slot * H + h) * (RWKV7_HEAD * RWKV7_HEAD)) + 256 * q;
    f32x4 S[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) S[m] = stream_load(sp + 64 * m + l);

    for (int t = t0; t < t1; ++t) {
        const size_t o = (size_t)t * C + (size_t)h * RWKV7_HEAD;
        const f32x4 r4 = tr::load4(r + o + 4 * c);
        const f32x4 k4 = tr::load4(k + o + 4 * c);
        const f32x4 a4 = tr::load4(a + o + 4 * c);
        const f32x4 b4 = tr::load4(b + o + 4 * c);
        const f32x4 wr = tr::load4(w + o + 4 * c);
        float vr[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) vr[m] = tr::to_f32(v[o + 16 * q + 4 * m + g]);
        f32x4 w4;
        w4.x = expf(-expf(wr.x));
        w4.y = expf(-expf(wr.y));
        w4.z = expf(-expf(wr.z));
        w4.w = expf(-expf(wr.w));
        float yq[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const float si = row16_sum(fast_dot4(a4, S[m]));  // sa of row 16q + 4m + g
            const float vi = vr[m];
            f32x4 x = S[m];
            x.x = fmaf(si, b4.x, fmaf(k4.x, vi, x.x * w4.x));
            x.y = fmaf(si, b4.y, fmaf(k4.y, vi, x.y * w4.y));
            x.z = fmaf(si, b4.z, fmaf(k4.z, vi, x.z * w4.z));
            x.w = fmaf(si, b4.w, fmaf(k4.w, vi, x.w * w4.w));
            S[m] = x;
            yq[m] = row16_sum(fast_dot4(x, r4));
        }
        // lane (g, c < 4) stores y of row 16q + 4c + g: the quarter's 16 values
        const float yv = c == 0 ? yq[0] : (c == 1 ? yq[1] : (c == 2 ? yq[2] : yq[3]));
        if (c < 4) y[o + 16 * q + 4 * c + g] = tr::from_f32(yv);
    }

#pragma unroll
    for (int m = 0; m < 4; ++m) stream_store(sp + 64 * m + l, S[m]);
}

}  // namespace

template <typename IO>
hipError_t launch_wkv7_seq(int nseq, int H, int T_uniform, const int32_t* cu_seqlens,
                           const int32_t* slot_idx, int pool_slots, int total_tokens,
                           float* state, const void* r, const void* w, const void* k,
                           const void* v, const void* a, const void* b, void* y,
                           hipStream_t stream)
{
    const unsigned grid = 4u * (unsigned)nseq * (unsigned)H;  // four quarter-unit blocks per (sequence, head)
    hipLaunchKernelGGL(wkv7_seq_kernel<IO>, dim3(grid), dim3(64), 0, stream,
                       H, T_uniform, cu_seqlens, slot_idx, pool_slots, total_tokens, state,
                       (const IO*)r, (const IO*)w, (const IO*)k, (const IO*)v, (const IO*)a,
                       (const IO*)b, (IO*)y);
    return hipGetLastError();
}

template hipError_t launch_wkv7_seq<float>(int, int, int, const int32_t*, const int32_t*, int, int,
                                           float*, const void*, const void*, const void*,
                                           const void*, const void*, const void*, void*, hipStream_t);
template hipError_t launch_wkv7_seq<bf16_t>(int, int, int, const int32_t*, const int32_t*, int, int,
                                            float*, const void*, const void*, const void*,
                                            const void*, const void*, const void*, void*, hipStream_t);
template hipError_t launch_wkv7_seq<f16_t>(int, int, int, const int32_t*, const int32_t*, int, int,
                                           float*, const void*, const void*, const void*,
                                           const void*, const void*, const void*, void*, hipStream_t);
