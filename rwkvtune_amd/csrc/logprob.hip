// Per-token log-probabilities of chosen tokens: out[r] = log_softmax(logits[r])[index[r]]
// without materialising the log-softmax (the selective_log_softmax of
// rwkvtune/training/grpo/utils.py:13-103, used by the GRPO log-prob recompute,
// grpo/lightning_module.py:1810-1964).
//
// One 256-thread block per row reads the row once with 16-byte loads, keeping an
// online (max, sum of exp(x - max)) per thread; the chosen logit is read once.
// Numerics follow the reference per dtype:
//   float32 logits:  out = x[i] - logsumexp(x)                       (fp32)
//   bf16 / fp16:     lse = logsumexp(float(x)) rounded to the dtype,
//                    out = round(float(x[i]) - float(lse))            (the dtype)
// (the reference computes torch.logsumexp(logits.float()).to(dtype) and
// subtracts in the dtype).  An index outside [0, V) gives NaN (the reference's
// gather raises instead; checking would cost a host synchronisation).
#include "common.hpp"

namespace {

constexpr int kT = 256;

__device__ __forceinline__ float block_reduce_max(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < kT / 64; ++i) s = fmaxf(s, red[i]);
    return s;
}

__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kT / 64; ++i) s += red[i];
    return s;
}

// 8 consecutive logits of a row as floats (16 or 32 bytes)
template <typename LT> struct Load8;
template <> struct Load8<float> {
    static __device__ __forceinline__ void get(const float* p, float (&x)[8]) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(p);
        const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
};
template <typename LT> struct Load8 {  // 16-bit types
    static __device__ __forceinline__ void get(const LT* p, float (&x)[8]) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const LT* e = reinterpret_cast<const LT*>(&u);
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = io_traits<LT>::to_f32(e[j]);
    }
};

// One pass over the row: each thread keeps a running (max, sum of exp(x - max))
// over its groups of 8 logits (rescaling the sum when the max grows), then the
// block combines the pairs.  vec: rows are 16-byte aligned and V % 8 == 0, else
// elements are read one by one.
template <typename LT>
__global__ __launch_bounds__(kT) void selective_logsoftmax_kernel(int V, const LT* __restrict__ logits, int64_t ld,
                                                                  const int64_t* __restrict__ index,
                                                                  LT* __restrict__ out, int vec)
{
    __shared__ float red[kT / 64];
    const int r = blockIdx.x, t = threadIdx.x;
    const LT* row = logits + (int64_t)r * ld;
    float m = -INFINITY, s = 0.f;
    for (int i0 = 8 * t; i0 < V; i0 += 8 * kT) {
        float x[8];
        if (vec && i0 + 8 <= V) {
            Load8<LT>::get(row + i0, x);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = (i0 + e < V) ? io_traits<LT>::to_f32(row[i0 + e]) : -INFINITY;
        }
        float mc = x[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) mc = fmaxf(mc, x[e]);
        if (mc > m) {
            s = (m == -INFINITY) ? 0.f : s * expf(m - mc);
            m = mc;
        }
        if (m != -INFINITY && m != INFINITY) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s += expf(x[e] - m);
        }
    }
    const float M = block_reduce_max(m, red);
    const float part = (m == -INFINITY || M == INFINITY) ? 0.f : s * expf(m - M);
    const float S = block_reduce_sum(part, red);
    if (t == 0) {
        // logsumexp as torch defines it: max + log(sum exp(x - max)); an all -inf
        // row gives -inf, a +inf max gives +inf
        const float lse = (M == -INFINITY || M == INFINITY) ? M : M + logf(S);
        const int64_t id = index[r];
        const float xs = (id >= 0 && id < V) ? io_traits<LT>::to_f32(row[id]) : NAN;
        float o;
        if (sizeof(LT) == 4) o = xs - lse;
        else o = xs - io_traits<LT>::to_f32(io_traits<LT>::from_f32(lse));
        out[r] = io_traits<LT>::from_f32(o);
    }
}

}  // namespace

template <typename LT>
hipError_t launch_selective_logsoftmax(int R, int V, const void* logits, int64_t ld, const int64_t* index, void* out,
                                       hipStream_t st)
{
    const int vec = (((uintptr_t)logits) & 15) == 0 && (V % 8) == 0 && ((ld * (int64_t)sizeof(LT)) % 16) == 0;
    hipLaunchKernelGGL((selective_logsoftmax_kernel<LT>), dim3(R), dim3(kT), 0, st, V, (const LT*)logits, ld, index,
                       (LT*)out, vec);
    return hipGetLastError();
}

template hipError_t launch_selective_logsoftmax<float>(int, int, const void*, int64_t, const int64_t*, void*,
                                                       hipStream_t);
template hipError_t launch_selective_logsoftmax<bf16_t>(int, int, const void*, int64_t, const int64_t*, void*,
                                                        hipStream_t);
template hipError_t launch_selective_logsoftmax<f16_t>(int, int, const void*, int64_t, const int64_t*, void*,
                                                       hipStream_t);
