// Token sampling on gfx950 without sorting the vocabulary.
//
// Semantics follow rwkvtune/inference/core.py (TokenSampler):
//   * ids above max_valid_id are banned (-inf)                      core.py:66-77, 171-181
//   * temperature < 1e-6 -> greedy argmax (lowest index on ties), logp =
//     log_softmax(banned logits)[token], no temperature / bias       core.py:80-83, 184-188
//   * logits / temperature, then logit_bias clamped to [-100, 100]   core.py:86-95, 191-204
//   * RULE_SINGLE (TokenSampler.sample, core.py:40-137): top_k > 0 samples the k
//     most probable tokens; else top_p < 1 keeps the sorted prefix up to and
//     including the first token whose cumulative probability exceeds top_p
//     (cutoff = #(cumsum <= p) + 1, core.py:119-131); logp = log(renormalised p + 1e-10);
//     non-finite probabilities fall back to the uniform distribution (core.py:102-108).
//   * RULE_BATCH (TokenSampler.sample_batch, core.py:142-236): top_k keeps the k
//     largest logits, then top_p keeps the sorted prefix with cumsum <= top_p and
//     always the first token (core.py:214-228); logp = log_softmax(filtered)[token].
//
// Design: one 1024-thread block per row; the row (V <= 65536) lives in registers,
// 64 values per thread, element i = j*1024 + tid.  The k-th largest value and the
// nucleus boundary are found by bisection over the order-preserving integer
// encoding of the float values (32 block reductions each), so no sort and no
// scratch memory.  Sampling draws u from a counter-based hash of (seed, row key,
// row counter) and walks the kept tokens in a fixed order (thread-major); ties at
// a threshold are kept together (the reference's sort keeps an arbitrary subset).
#include "common.hpp"

namespace {

constexpr int kT = 1024;
constexpr int kVPT = 64;  // values per thread
constexpr int kW = kT / 64;

enum { RULE_BATCH = 0, RULE_SINGLE = 1 };

__device__ __forceinline__ uint32_t okey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {  // SplitMix64 finaliser (Steele et al. 2014)
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// uniform in [0, 1) with 24 random bits
__device__ __forceinline__ float uniform01(uint64_t seed, uint64_t key, uint64_t ctr) {
    uint64_t z = mix64(seed + 0x9e3779b97f4a7c15ull);
    z = mix64(z ^ (key * 0xd1342543de82ef95ull + 0x632be59bd9b4e019ull));
    z = mix64(z ^ (ctr * 0x9e3779b97f4a7c15ull + 0x2545f4914f6cdd1dull));
    return (float)(z >> 40) * (1.0f / 16777216.0f);
}

template <typename T>
__device__ __forceinline__ T wave_reduce_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_reduce_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

struct Red {
    float f[kW];
    unsigned u[kW];
    double d[kW];
};

__device__ float block_sum_f(float v, Red* red) {
    v = wave_reduce_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red->f[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kW; ++i) s += red->f[i];
    return s;
}

__device__ float block_max_f(float v, Red* red) {
    v = wave_reduce_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red->f[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = -INFINITY;
#pragma unroll
    for (int i = 0; i < kW; ++i) s = fmaxf(s, red->f[i]);
    return s;
}

__device__ unsigned block_sum_u(unsigned v, Red* red) {
    v = wave_reduce_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red->u[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned s = 0;
#pragma unroll
    for (int i = 0; i < kW; ++i) s += red->u[i];
    return s;
}

// argmax with the lowest index on ties: pack (key, ~index) into 64 bits
__device__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    unsigned long long s = 0;
#pragma unroll
    for (int i = 0; i < kW; ++i) s = red[i] > s ? red[i] : s;
    return s;
}

template <typename LT>
__global__ __launch_bounds__(kT) void sample_kernel(
    int M, int V, const LT* __restrict__ logits, int64_t ld, int rule, int max_valid_id,
    const float* __restrict__ temperature, const float* __restrict__ top_p,
    const int32_t* __restrict__ top_k, const int32_t* __restrict__ bias_off,
    const int32_t* __restrict__ bias_ids, const float* __restrict__ bias_val,
    const uint8_t* __restrict__ active, uint64_t seed, const int64_t* __restrict__ rng_key,
    const int32_t* __restrict__ rng_ctr, int64_t* __restrict__ out_tok, float* __restrict__ out_logp)
{
    typedef io_traits<LT> tr;
    __shared__ Red red;
    __shared__ unsigned long long red64[kW];
    __shared__ float thread_mass[kT];
    __shared__ int pick;
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;  // whole block
    const int tid = threadIdx.x;
    const LT* lg = logits + (size_t)row * ld;
    const int vmax = max_valid_id < V - 1 ? max_valid_id : V - 1;

    float x[kVPT];
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        const int i = j * kT + tid;
        x[j] = (i <= vmax) ? tr::to_f32(lg[i]) : -INFINITY;  // banned and padding: -inf
    }

    const float temp = temperature[row];
    if (!(temp >= 1e-6f)) return;  // greedy rows belong to greedy_kernel
    // temperature, then logit bias (clamped), core.py:86-95
#pragma unroll
    for (int j = 0; j < kVPT; ++j) x[j] = x[j] / temp;
    if (bias_off != nullptr) {
        const int b0 = bias_off[row], b1 = bias_off[row + 1];
        for (int q = b0; q < b1; ++q) {
            const int id = bias_ids[q];
            if (id >= 0 && id < V && (id % kT) == tid) {
                const float bv = fminf(100.f, fmaxf(-100.f, bias_val[q]));
                // static register index: unrolled select
#pragma unroll
                for (int j = 0; j < kVPT; ++j)
                    if (j == id / kT) x[j] += bv;
            }
        }
    }

    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) mm = fmaxf(mm, x[j]);
    const float mx = block_max_f(mm, &red);
    // From here on a token is its key: the bit pattern of its unnormalised
    // probability q = exp(l - max) >= 0 (0 for banned and padding entries).  For
    // non-negative floats the bit pattern orders like the value, so keys order
    // tokens like their logits, q is read back by reinterpreting the key (no
    // instruction, nothing for the compiler to hoist), and one 32-bit register
    // per token keeps the row resident.
    uint32_t key[kVPT];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        const float q = (x[j] == -INFINITY) ? 0.f : expf(x[j] - mx);
        key[j] = __float_as_uint(q);  // padding: q = 0
        s += q;
    }
    const float Z = block_sum_f(s, &red);
    const bool uniform = !(mx > -INFINITY) || !(mx < INFINITY) || !(Z < INFINITY) || !(Z > 0.f);

    // kept set: key >= lo (lo = 1: every token with non-zero probability)
    uint32_t lo = 1;
    float W = Z;  // unnormalised kept mass
    const int k = top_k[row];
    const float p = top_p[row];
    if (!uniform && k > 0 && k < V) {
        // largest K with count(key >= K) >= k  (the k-th largest value)
        uint32_t K = 0;
        for (int bit = 31; bit >= 0; --bit) {
            const uint32_t cand = K | (1u << bit);
            unsigned c = 0;
#pragma unroll
            for (int j = 0; j < kVPT; ++j) c += key[j] >= cand ? 1u : 0u;
            if (block_sum_u(c, &red) >= (unsigned)k) K = cand;
        }
        lo = K > 1u ? K : 1u;
        float sk = 0.f;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) sk += key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
        W = block_sum_f(sk, &red);
    }
    const bool nucleus = !uniform && p < 1.0f && (rule == RULE_BATCH || k <= 0);
    if (nucleus) {
        // largest K' with mass(key >= max(K', lo)) > p * W: the key of the token
        // whose inclusion crosses p.  The mass counts only top-k survivors, so the
        // predicate holds for every K' <= lo and the bisection starts from 0.
        const float target = p * W;
        uint32_t K = 0;
        for (int bit = 31; bit >= 0; --bit) {
            const uint32_t cand = K | (1u << bit);
            const uint32_t thr = cand > lo ? cand : lo;
            float ms = 0.f;
#pragma unroll
            for (int j = 0; j < kVPT; ++j) ms += key[j] >= thr ? __uint_as_float(key[j]) : 0.f;
            if (block_sum_f(ms, &red) > target) K = cand;
        }
        // RULE_SINGLE keeps the crossing token, RULE_BATCH stops before it but
        // always keeps the most probable token (q = 1)
        uint32_t nlo = (rule == RULE_SINGLE) ? K : K + 1u;
        const uint32_t top = __float_as_uint(1.0f);
        if (nlo > top) nlo = top;
        lo = nlo > lo ? nlo : lo;
        float sk = 0.f;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) sk += key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
        W = block_sum_f(sk, &red);
    }

    const float u = uniform01(seed, (uint64_t)rng_key[row], (uint64_t)(uint32_t)rng_ctr[row]);
    if (uniform) {  // non-finite probabilities: uniform over the vocabulary (core.py:102-108)
        if (tid == 0) {
            int t = (int)(u * (float)V);
            out_tok[row] = t < V ? t : V - 1;
            out_logp[row] = logf(1.0f / (float)V + 1e-10f);
        }
        return;
    }
    // inverse-CDF draw over the kept tokens in thread-major order
    float tm = 0.f;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) tm += key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
    thread_mass[tid] = tm;
    if (tid == 0) pick = -1;
    __syncthreads();
    // inclusive scan of the 1024 thread masses (Hillis-Steele in LDS)
    float acc = tm;
    for (int o = 1; o < kT; o <<= 1) {
        const float add = tid >= o ? thread_mass[tid - o] : 0.f;
        __syncthreads();
        acc += add;
        thread_mass[tid] = acc;
        __syncthreads();
    }
    // [before, acc) of consecutive threads tile [0, total) exactly
    const float total = thread_mass[kT - 1];
    const float target = u * total;
    const float before = tid > 0 ? thread_mass[tid - 1] : 0.f;
    if (tm > 0.f && target >= before && (target < acc || acc >= total)) {
        // fully unrolled (no early exit) so key[] stays in registers
        float c = before;
        int chosen = -1;
        bool done = false;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) {
            const float w = key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
            if (!done && w > 0.f) {
                chosen = j * kT + tid;
                c += w;
                done = c > target;
            }
        }
        atomicMax(&pick, chosen);
    }
    __syncthreads();
    const int tok = pick;
    if (tok >= 0 && tid == (tok % kT)) {
        uint32_t kq = 0;
#pragma unroll
        for (int j = 0; j < kVPT; ++j)
            if (j == tok / kT) kq = key[j];
        const float q = __uint_as_float(kq);
        out_tok[row] = tok;
        out_logp[row] = (rule == RULE_SINGLE) ? logf(q / W + 1e-10f) : logf(q) - logf(W);
    }
}


// Greedy rows (temperature < 1e-6, core.py:80-83, 184-188): argmax of the banned
// logits with the lowest index on ties, logp = log_softmax(banned logits)[token].
// A kernel of its own: sharing one kernel with the sampling path doubles its
// register footprint.
template <typename LT>
__global__ __launch_bounds__(kT) void greedy_kernel(
    int M, int V, const LT* __restrict__ logits, int64_t ld, int max_valid_id,
    const float* __restrict__ temperature, const uint8_t* __restrict__ active,
    int64_t* __restrict__ out_tok, float* __restrict__ out_logp)
{
    typedef io_traits<LT> tr;
    __shared__ Red red;
    __shared__ unsigned long long red64[kW];
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;
    if (temperature[row] >= 1e-6f) return;  // sampled rows belong to sample_kernel
    const int tid = threadIdx.x;
    const LT* lg = logits + (size_t)row * ld;
    const int vmax = max_valid_id < V - 1 ? max_valid_id : V - 1;
    float x[kVPT];
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        const int i = j * kT + tid;
        x[j] = (i <= vmax) ? tr::to_f32(lg[i]) : -INFINITY;
    }
    // padding is -inf at the highest indices, so it never wins a tie
    unsigned long long best = 0;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        const unsigned i = (unsigned)(j * kT + tid);
        const unsigned long long c = ((unsigned long long)okey(x[j]) << 32) | (unsigned long long)(0xffffffffu - i);
        best = c > best ? c : best;
    }
    best = block_max_u64(best, red64);
    const int tok = (int)(0xffffffffu - (unsigned)(best & 0xffffffffull));
    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) mm = fmaxf(mm, x[j]);
    const float mx = block_max_f(mm, &red);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) s += (x[j] == -INFINITY) ? 0.f : expf(x[j] - mx);
    const float Z = block_sum_f(s, &red);
    if (tid == 0) {
        out_tok[row] = tok;
        // the argmax value is mx unless every logit is -inf / NaN
        out_logp[row] = (mx == -INFINITY) ? -INFINITY : -logf(Z);
    }
}

// Repetition penalty, in place, once per occurrence of each id in the row's
// history (grpo_batch_generator.py:25-42): logit / p if logit > 0 else logit * p.
// The history of row m is hist[hist_start[m] .. + hist_len[m]) followed by
// hist2[hist2_start[m] .. + hist2_len[m]) (second segment nullable).  Repeated
// applications to one logit commute (the sign never changes), so the atomic
// updates give the same result in any order.
__global__ __launch_bounds__(256) void rep_penalty_kernel(
    int M, int V, float* __restrict__ logits, int64_t ld, float penalty,
    const int32_t* __restrict__ hist, const int64_t* __restrict__ hist_start,
    const int32_t* __restrict__ hist_len, const int32_t* __restrict__ hist2,
    const int64_t* __restrict__ hist2_start, const int32_t* __restrict__ hist2_len,
    const uint8_t* __restrict__ active)
{
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;
    float* lg = logits + (size_t)row * ld;
    auto apply = [&](int id) {
        if (id < 0 || id >= V) return;
        unsigned int* addr = reinterpret_cast<unsigned int*>(lg + id);
        unsigned int old = *addr, assumed;
        do {
            assumed = old;
            const float f = __uint_as_float(assumed);
            const float nf = f > 0.f ? f / penalty : f * penalty;
            old = atomicCAS(addr, assumed, __float_as_uint(nf));
        } while (old != assumed);
    };
    const int64_t a0 = hist_start[row];
    const int64_t a1 = a0 + hist_len[row];
    for (int64_t q = a0 + threadIdx.x; q < a1; q += blockDim.x) apply(hist[q]);
    if (hist2 != nullptr) {
        const int64_t b0 = hist2_start[row];
        const int64_t b1 = b0 + hist2_len[row];
        for (int64_t q = b0 + threadIdx.x; q < b1; q += blockDim.x) apply(hist2[q]);
    }
}

}  // namespace

template <typename LT>
hipError_t launch_sample(int M, int V, const void* logits, int64_t ld, int rule, int max_valid_id,
                         const float* temperature, const float* top_p, const int32_t* top_k,
                         const int32_t* bias_off, const int32_t* bias_ids, const float* bias_val,
                         const uint8_t* active, uint64_t seed, const int64_t* rng_key,
                         const int32_t* rng_ctr, int64_t* out_tok, float* out_logp, hipStream_t st)
{
    hipLaunchKernelGGL(greedy_kernel<LT>, dim3(M), dim3(kT), 0, st, M, V, (const LT*)logits, ld, max_valid_id,
                       temperature, active, out_tok, out_logp);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(sample_kernel<LT>, dim3(M), dim3(kT), 0, st, M, V, (const LT*)logits, ld, rule,
                       max_valid_id, temperature, top_p, top_k, bias_off, bias_ids, bias_val, active, seed,
                       rng_key, rng_ctr, out_tok, out_logp);
    return hipGetLastError();
}

template hipError_t launch_sample<float>(int, int, const void*, int64_t, int, int, const float*, const float*,
                                         const int32_t*, const int32_t*, const int32_t*, const float*,
                                         const uint8_t*, uint64_t, const int64_t*, const int32_t*, int64_t*,
                                         float*, hipStream_t);
template hipError_t launch_sample<bf16_t>(int, int, const void*, int64_t, int, int, const float*, const float*,
                                          const int32_t*, const int32_t*, const int32_t*, const float*,
                                          const uint8_t*, uint64_t, const int64_t*, const int32_t*, int64_t*,
                                          float*, hipStream_t);
template hipError_t launch_sample<f16_t>(int, int, const void*, int64_t, int, int, const float*, const float*,
                                         const int32_t*, const int32_t*, const int32_t*, const float*,
                                         const uint8_t*, uint64_t, const int64_t*, const int32_t*, int64_t*,
                                         float*, hipStream_t);

hipError_t launch_rep_penalty(int M, int V, float* logits, int64_t ld, float penalty, const int32_t* hist,
                              const int64_t* hist_start, const int32_t* hist_len, const int32_t* hist2,
                              const int64_t* hist2_start, const int32_t* hist2_len, const uint8_t* active,
                              hipStream_t st)
{
    hipLaunchKernelGGL(rep_penalty_kernel, dim3(M), dim3(256), 0, st, M, V, logits, ld, penalty, hist, hist_start,
                       hist_len, hist2, hist2_start, hist2_len, active);
    return hipGetLastError();
}

int sampler_max_vocab() { return kT * kVPT; }
