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
//   * RULE_MIXIN (GenerationMixin.generate, rwkvtune/models/generation_mixin.py:
//     188-211): top_k keeps the k largest, then - only when 0 < top_p < 1 - the
//     renormalised nucleus up to and including the crossing token (the shifted
//     cumsum > top_p mask); logp = log(renormalised p + 1e-10).
//
// Design: one 1024-thread block per row; the row (V <= 65536) lives in registers,
// 64 values per thread, read with 16-byte loads (layout at load_row).  A token is the bit pattern of
// its unnormalised probability q = exp(l - max) (orders like the logit).  The
// k-th largest key and the nucleus boundary are found by a three-level radix
// select over the keys (11, 10 and 10 bits: 1024 LDS bins per level, built with
// LDS atomics, then one block scan from the top bin down), counting tokens for
// top-k and summing their probability in 31-bit fixed point (q * 2^31, 64-bit
// sums: integer, so the result does not depend on the order of the atomics) for
// top-p.  Sampling draws u from a counter-based hash of (seed, row key, row
// counter) and walks the kept tokens in a fixed order (thread-major); ties at a
// threshold are kept together (the reference's sort keeps an arbitrary subset).
#include "common.hpp"

namespace {

// sample_kernel and greedy_kernel: 1024 threads x 64 values
constexpr int kT = 1024;
constexpr int kVPT = 64;  // values per thread
constexpr int kTG = 1024, kVPTG = 64;
constexpr int kWMax = 16;  // waves of the larger block
constexpr int kBins = 1024;  // radix bins per level (one per thread)

enum { RULE_BATCH = 0, RULE_SINGLE = 1, RULE_MIXIN = 2 };

// Row layout in registers: thread t holds x[8c + e] = element 8192 c + 8 t + e
// (c < 8, e < 8), so each group of 8 is one 16-byte load of a 16-bit row.
constexpr int kGroup = 8, kStride = kT * kGroup;
__device__ __forceinline__ int elem_of(int j, int tid) { return (j / kGroup) * kStride + tid * kGroup + (j % kGroup); }
__device__ __forceinline__ int owner_of(int i) { return (i % kStride) / kGroup; }
__device__ __forceinline__ int slot_of(int i) { return (i / kStride) * kGroup + (i % kGroup); }

// the row's values with entries past vmax (banned ids and padding) as -inf.  No
// load depends on a condition (a conditional load is waited on where it stands,
// which serialises the row's loads): on an aligned row with V % 8 == 0 every group
// of 8 is wholly inside the row or wholly past it, and is one 16-byte load (two for
// float32) of the group or, past the row, of group 0; otherwise every element is
// one load from an index clamped to the row.  The masks are selects afterwards.
template <typename LT>
__device__ __forceinline__ void load_row(const LT* lg, int V, int vmax, float (&x)[kVPT]) {
    typedef io_traits<LT> tr;
    const int tid = threadIdx.x;
    if ((((uintptr_t)lg) & 15) == 0 && V % kGroup == 0) {
        f32x4 a[kVPT / kGroup], b[kVPT / kGroup];
#pragma unroll
        for (int c = 0; c < kVPT / kGroup; ++c) {
            const int i0 = c * kStride + tid * kGroup;
            const LT* p = lg + (i0 < V ? i0 : 0);
            a[c] = tr::load4(p);
            b[c] = tr::load4(p + 4);
        }
#pragma unroll
        for (int c = 0; c < kVPT / kGroup; ++c) {
            const int i0 = c * kStride + tid * kGroup;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[c * kGroup + e] = i0 + e <= vmax ? a[c][e] : -INFINITY;
                x[c * kGroup + 4 + e] = i0 + 4 + e <= vmax ? b[c][e] : -INFINITY;
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < kVPT / kGroup; ++c) {
#pragma unroll
            for (int e = 0; e < kGroup; ++e) {
                const int i = c * kStride + tid * kGroup + e;
                const float v = tr::to_f32(lg[i < V ? i : V - 1]);
                x[c * kGroup + e] = i <= vmax ? v : -INFINITY;
            }
        }
    }
}

// exp(x) as one v_exp_f32 of x * log2(e) (a few ulp: sampling weights)
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

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
    float f[kWMax];
};

__device__ float block_sum_f(float v, Red* red) {
    v = wave_reduce_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red->f[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s += red->f[i];
    return s;
}

__device__ float block_max_f(float v, Red* red) {
    v = wave_reduce_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red->f[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = -INFINITY;
#pragma unroll
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s = fmaxf(s, red->f[i]);
    return s;
}

// inclusive prefix sum over the block in thread order (wave scans, then the
// wave totals); `wsum` holds one entry per wave
template <typename T>
__device__ T block_incl_scan(T v, T* wsum) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T n = __shfl_up(v, o, 64);
        if (lane >= o) v += n;
    }
    __syncthreads();  // wsum of a previous scan has been read
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    T off = 0;
    for (int i = 0; i < w; ++i) off += wsum[i];
    return v + off;
}

// Inclusive prefix sum over the block in thread order, and the exclusive one
// bit-identical to the previous thread's inclusive sum (lane 0 takes the wave
// offset, which is the previous wave's last inclusive sum by commutativity), so
// the intervals [excl, incl) of consecutive threads tile [0, total) with no gap
// or overlap in float arithmetic.  `wsum` holds one entry per wave.
__device__ float block_scan_tiled(float v, float* wsum, float& excl) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float n = __shfl_up(v, o, 64);
        if (lane >= o) v += n;
    }
    const float prev = __shfl_up(v, 1, 64);
    __syncthreads();  // wsum of a previous scan has been read
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    float off = 0.f;
    for (int i = 0; i < w; ++i) off += wsum[i];
    excl = lane == 0 ? off : prev + off;
    return v + off;
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
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) s = red[i] > s ? red[i] : s;
    return s;
}

// One level of the radix select.  Tokens with key >= lo whose bits above
// `shift + 10` equal `prefix` (all of them when `first`) are binned by bits
// shift .. shift+9 of the key; a bin holds their count (COUNT) or their mass in
// fixed point (q * 2^31, truncated).  Walking the bins from the top, starting
// from `above` (the amount in the higher bins of earlier levels), the selected
// bin is the one where the running total first exceeds `target` (COUNT: first
// reaches it).  `frac` > 0 sets target = frac * (this level's total) first (the
// nucleus: the first level bins every kept token).  Returns the bin; `above`
// becomes the amount in the bins above it.
template <bool COUNT>
__device__ uint32_t radix_level(const uint32_t (&key)[kVPT], uint32_t lo, int shift, uint32_t prefix, bool first,
                                unsigned long long& above, unsigned long long& target, float frac,
                                unsigned long long* bins, unsigned long long* wsum, int* pick_bin,
                                unsigned long long* pick_val) {
    const int tid = threadIdx.x;
    static_assert(kBins == kT, "one bin per thread");
    bins[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        const uint32_t kj = key[j];
        const bool in = kj >= lo && (first || (kj >> (shift + 10)) == prefix);
        if (in) {
            const unsigned long long add =
                COUNT ? 1ull : (unsigned long long)(uint32_t)(__uint_as_float(kj) * 2147483648.0f);
            atomicAdd(&bins[(kj >> shift) & 1023], add);
        }
    }
    __syncthreads();
    const uint32_t b = kBins - 1 - tid;  // thread 0 takes the top bin
    const unsigned long long val = bins[b];
    const unsigned long long incl = block_incl_scan(val, wsum);
    if (frac > 0.f) {
        if (tid == kT - 1) *pick_val = incl;  // the level's total
        __syncthreads();
        target = (unsigned long long)((double)frac * (double)(*pick_val));
        __syncthreads();
    }
    const unsigned long long lo_sum = above + incl - val, hi_sum = above + incl;
    const bool hit = COUNT ? (hi_sum >= target && lo_sum < target) : (hi_sum > target && lo_sum <= target);
    if (hit) {
        *pick_bin = (int)b;
        *pick_val = lo_sum;
    }
    __syncthreads();
    above = *pick_val;
    const uint32_t r = (uint32_t)*pick_bin;
    __syncthreads();  // pick_* are rewritten by the next level
    return r;
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
    __shared__ Red red;
    __shared__ unsigned long long bins[kBins];
    __shared__ unsigned long long wsum[kWMax];
    __shared__ float fsum[kWMax];
    __shared__ int pick_bin;
    __shared__ unsigned long long pick_val;
    __shared__ int pick;
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;  // whole block
    const int tid = threadIdx.x;
    const LT* lg = logits + (size_t)row * ld;
    const int vmax = max_valid_id < V - 1 ? max_valid_id : V - 1;

    const float temp = temperature[row];
    if (!(temp >= 1e-6f)) return;  // greedy rows belong to greedy_kernel
    float x[kVPT];
    load_row(lg, V, vmax, x);  // banned and padding: -inf
    // temperature (a multiply by its reciprocal: within an ulp of the division),
    // then logit bias (clamped), core.py:86-95
    if (temp != 1.0f) {
        const float it = 1.0f / temp;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) x[j] *= it;
    }
    if (bias_off != nullptr) {
        const int b0 = bias_off[row], b1 = bias_off[row + 1];
        for (int q = b0; q < b1; ++q) {
            const int id = bias_ids[q];
            if (id >= 0 && id < V && owner_of(id) == tid) {
                const float bv = fminf(100.f, fmaxf(-100.f, bias_val[q]));
                // static register index: unrolled select
#pragma unroll
                for (int j = 0; j < kVPT; ++j)
                    if (j == slot_of(id)) x[j] += bv;
            }
        }
    }

    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) mm = fmaxf(mm, x[j]);
    const float mx = block_max_f(mm, &red);
    // From here on a token is its key: the bit pattern of q = exp(l - max) >= 0
    // (0 for banned and padding entries), which orders like the logit; q is read
    // back by reinterpreting the key, and one register per token keeps the row.
    uint32_t key[kVPT];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        // a NaN logit stays NaN here (the compare is false), so Z turns NaN and
        // the row takes the uniform fallback, as the reference's isnan(probs) does
        const float e = fast_exp(x[j] - mx);
        const float q = (x[j] == -INFINITY) ? 0.f : (e > 1.0f ? 1.0f : e);
        key[j] = __float_as_uint(q);
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
        // the k-th largest key: the highest K with count(key >= K) >= k
        unsigned long long above = 0, target = (unsigned long long)k;
        const uint32_t b1 = radix_level<true>(key, 0u, 20, 0u, true, above, target, 0.f, bins, wsum, &pick_bin,
                                              &pick_val);
        const uint32_t b2 = radix_level<true>(key, 0u, 10, b1, false, above, target, 0.f, bins, wsum, &pick_bin,
                                              &pick_val);
        const uint32_t b3 = radix_level<true>(key, 0u, 0, (b1 << 10) | b2, false, above, target, 0.f, bins, wsum,
                                              &pick_bin, &pick_val);
        const uint32_t K = (b1 << 20) | (b2 << 10) | b3;
        lo = K > 1u ? K : 1u;
        float sk = 0.f;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) sk += key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
        W = block_sum_f(sk, &red);
    }
    const bool nucleus = !uniform && p < 1.0f &&
                         (rule == RULE_BATCH || (rule == RULE_MIXIN && p > 0.f) || (rule == RULE_SINGLE && k <= 0));
    if (nucleus) {
        // the key of the token whose inclusion crosses p: the highest K' with
        // mass(key >= max(K', lo)) > p * mass(key >= lo), in fixed point
        unsigned long long above = 0, target = 0;
        const uint32_t b1 = radix_level<false>(key, lo, 20, 0u, true, above, target, fmaxf(p, 1e-30f), bins, wsum,
                                               &pick_bin, &pick_val);
        const uint32_t b2 = radix_level<false>(key, lo, 10, b1, false, above, target, 0.f, bins, wsum, &pick_bin,
                                               &pick_val);
        const uint32_t b3 = radix_level<false>(key, lo, 0, (b1 << 10) | b2, false, above, target, 0.f, bins, wsum,
                                               &pick_bin, &pick_val);
        const uint32_t K = (b1 << 20) | (b2 << 10) | b3;
        // RULE_SINGLE and RULE_MIXIN keep the crossing token, RULE_BATCH stops
        // before it but always keeps the most probable token (q = 1)
        uint32_t nlo = (rule == RULE_BATCH) ? K + 1u : K;
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
    if (tid == 0) pick = -1;
    float before;
    // [before, acc) of consecutive threads tile [0, total) exactly, so exactly one
    // thread with kept mass owns the target (a rounded acc - tm could leave a gap
    // that no thread owns, and the draw unwritten)
    const float acc = block_scan_tiled(tm, fsum, before);
    // every wave reads fsum[0 .. w-1] at the end of the scan: wait for all of
    // them before fsum[0] is reused for the total
    __syncthreads();
    if (tid == kT - 1) fsum[0] = acc;             // total
    __syncthreads();
    const float total = fsum[0];
    const float target = u * total;
    if (tm > 0.f && target >= before && (target < acc || acc >= total)) {
        // fully unrolled (no early exit) so key[] stays in registers
        float c = before;
        int chosen = -1;
        bool done = false;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) {
            const float w = key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
            if (!done && w > 0.f) {
                chosen = elem_of(j, tid);
                c += w;
                done = c > target;
            }
        }
        atomicMax(&pick, chosen);
    }
    __syncthreads();
    if (pick < 0) {
        // not reached when the intervals tile (the total is finite and > 0 here);
        // kept as a deterministic guard: the lowest kept id
        if (tid == 0) pick_bin = 0x7fffffff;
        __syncthreads();
        int first = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < kVPT; ++j)
            if (key[j] >= lo) first = min(first, elem_of(j, tid));
        if (first != 0x7fffffff) atomicMin(&pick_bin, first);
        __syncthreads();
        if (tid == 0 && pick_bin != 0x7fffffff) pick = pick_bin;
        __syncthreads();
    }
    const int tok = pick;
    if (tok >= 0 && tid == owner_of(tok)) {
        uint32_t kq = 0;
#pragma unroll
        for (int j = 0; j < kVPT; ++j)
            if (j == slot_of(tok)) kq = key[j];
        const float q = __uint_as_float(kq);
        out_tok[row] = tok;
        out_logp[row] = (rule == RULE_BATCH) ? logf(q) - logf(W) : logf(q / W + 1e-10f);
    }
}

// Greedy rows (temperature < 1e-6, core.py:80-83, 184-188): argmax of the banned
// logits with the lowest index on ties, logp = log_softmax(banned logits)[token].
// A kernel of its own: sharing one kernel with the sampling path doubles its
// register footprint.
template <typename LT>
__global__ __launch_bounds__(kTG) void greedy_kernel(
    int M, int V, const LT* __restrict__ logits, int64_t ld, int max_valid_id,
    const float* __restrict__ temperature, const uint8_t* __restrict__ active,
    int64_t* __restrict__ out_tok, float* __restrict__ out_logp)
{
    typedef io_traits<LT> tr;
    __shared__ Red red;
    __shared__ unsigned long long red64[kWMax];
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;
    if (temperature[row] >= 1e-6f) return;  // sampled rows belong to sample_kernel
    const int tid = threadIdx.x;
    const LT* lg = logits + (size_t)row * ld;
    const int vmax = max_valid_id < V - 1 ? max_valid_id : V - 1;
    float x[kVPTG];
#pragma unroll
    for (int j = 0; j < kVPTG; ++j) {
        const int i = j * kTG + tid;
        const float v = tr::to_f32(lg[i < V ? i : V - 1]);  // unconditional load (see load_row)
        x[j] = i <= vmax ? v : -INFINITY;
    }
    // padding is -inf at the highest indices, so it never wins a tie
    unsigned long long best = 0;
#pragma unroll
    for (int j = 0; j < kVPTG; ++j) {
        const unsigned i = (unsigned)(j * kTG + tid);
        const unsigned long long c = ((unsigned long long)okey(x[j]) << 32) | (unsigned long long)(0xffffffffu - i);
        best = c > best ? c : best;
    }
    best = block_max_u64(best, red64);
    const int tok = (int)(0xffffffffu - (unsigned)(best & 0xffffffffull));
    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kVPTG; ++j) mm = fmaxf(mm, x[j]);
    const float mx = block_max_f(mm, &red);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVPTG; ++j) s += (x[j] == -INFINITY) ? 0.f : expf(x[j] - mx);
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
    hipLaunchKernelGGL(greedy_kernel<LT>, dim3(M), dim3(kTG), 0, st, M, V, (const LT*)logits, ld, max_valid_id,
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
static_assert(kT * kVPT == kTG * kVPTG, "both kernels cover the same vocabulary");
