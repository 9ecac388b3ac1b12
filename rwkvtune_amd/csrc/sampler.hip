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
// Design: one 1024-thread block per row; the row (V <= 65536) lives in
// registers, 64 values per thread, read with 16-byte loads (layout at load_row);
// nothing is sorted.
//   * 16-bit logits without logit_bias (sample16_kernel, the rollout's case): a
//     16-bit logit takes at most 65,536 values, so an LDS histogram of the row's
//     values (one atomic per token) is an exact sort.  Counts and masses
//     (count x q(value), q = exp(l - max) in 31-bit fixed point, 64-bit sums:
//     order-independent) are read per 64-value segment with one exponential
//     per occupied value; top-k and the nucleus are found by a scan of the
//     segment totals and a one-wave walk of the crossing segment; the draw
//     picks a value by an integer inverse CDF over the kept values, then the
//     j-th token of that value.
//   * other rows (float32 logits, logit_bias: sample_kernel): a token is the
//     bit pattern of q, which orders like the logit; the k-th largest key and
//     the nucleus boundary are found by a three-level radix select (2048, 2048
//     and 256 LDS bins, the two finer levels over a compacted candidate list),
//     the draw by an inverse CDF over the kept tokens in thread-major order.
// Random draws come from a counter-based hash of (seed, row key, row counter).
// Ties at a threshold are kept together (the reference's sort keeps an
// arbitrary subset).
#include "common.hpp"

namespace {

// sample16_kernel, sample_kernel and greedy_kernel: 1024 threads x 64 values
constexpr int kT = 1024;
constexpr int kVPT = 64;  // values per thread
constexpr int kTG = 1024, kVPTG = 64;
constexpr int kWMax = 16;  // waves of the larger block

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

// Threshold search.  The k-th largest key (top-k: counting) or the key of the
// token whose inclusion crosses p of the kept mass (top-p: q in 31-bit fixed
// point, summed in 64-bit integers, so the result does not depend on the order
// of the atomics) is found in three radix levels over bits 19..29, 8..18 and
// 0..7 of the key (keys are < 2^30: q <= 1): 2048, 2048 and 256 LDS bins.  The
// first level bins every candidate token from registers (for the nucleus without
// top-k, during the exponential pass); the candidates in the selected bin are
// then appended to a list in LDS, each wave to its own region, and the two finer
// levels bin the list only.  When a wave has more candidates than its region
// holds (a crowded bin: ties, flat rows), both finer levels bin the registers
// again instead.
constexpr int kSelBins = 2048;
constexpr int kListPerWave = 512;
constexpr int kWaves = kT / 64;

struct SelShared {
    unsigned long long bins[kSelBins];
    uint32_t list[kWaves * kListPerWave];
    unsigned long long wsum[kWMax];
    unsigned long long pick_val, total;
    int cnt[kWaves];
    int pick_bin;
};

// a token's amount in a bin: 1 (COUNT) or q * 2^31 truncated (q <= 1)
template <bool COUNT>
__device__ __forceinline__ unsigned long long sel_amount(uint32_t key) {
    return COUNT ? 1ull : (unsigned long long)(uint32_t)(__uint_as_float(key) * 2147483648.0f);
}

// Bin the register keys >= lo whose bits from pshift up equal prefix by bits
// shift .. of the key (mask: bin count - 1).
template <bool COUNT>
__device__ __forceinline__ void bin_registers(const uint32_t (&key)[kVPT], uint32_t lo, int shift, uint32_t mask,
                                              int pshift, uint32_t prefix, unsigned long long* bins) {
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        // opaque copy: the per-token compares and amounts are otherwise hoisted out of
        // the caller's level loop, 64 of each held in registers (spills)
        uint32_t kj = key[j];
        asm volatile("" : "+v"(kj));
        if (kj >= lo && (kj >> pshift) == prefix) atomicAdd(&bins[(kj >> shift) & mask], sel_amount<COUNT>(kj));
    }
}

// The same over the candidate list (every entry is >= lo): each wave bins its own region.
template <bool COUNT>
__device__ __forceinline__ void bin_list(SelShared& sh, int shift, uint32_t mask, int pshift, uint32_t prefix) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n = min(sh.cnt[w], kListPerWave);
    const uint32_t* src = sh.list + w * kListPerWave;
    for (int i = lane; i < n; i += 64) {
        const uint32_t kj = src[i];
        if ((kj >> pshift) == prefix) atomicAdd(&sh.bins[(kj >> shift) & mask], sel_amount<COUNT>(kj));
    }
}

// Append the register keys >= lo of first-level bin b1 to the wave's list region
// (positions past the region are counted, not written); the count goes to cnt[wave].
__device__ __forceinline__ void compact(const uint32_t (&key)[kVPT], uint32_t lo, uint32_t b1, SelShared& sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    uint32_t* dst = sh.list + w * kListPerWave;
    int n = 0;  // wave-uniform
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        uint32_t kj = key[j];
        asm volatile("" : "+v"(kj));
        const bool in = kj >= lo && (kj >> 19) == b1;
        const unsigned long long m = __ballot(in);
        if (m != 0ull) {
            const int pos = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            if (in && pos < kListPerWave) dst[pos] = kj;
            n += __popcll(m);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (lane == 0) sh.cnt[w] = n;
}

// Walk the nb bins from the top, starting from `above` (the amount in the bins
// above this level's range): the selected bin is the one where the running total
// first reaches `target` (COUNT) or first exceeds it (mass).  frac > 0 sets
// target = frac * (this level's total) first.  Returns the bin (0 when no bin
// qualifies); `above` becomes the amount above it.  Thread t reads bins
// nb-1-2t and nb-2-2t.
template <bool COUNT>
__device__ uint32_t scan_pick(SelShared& sh, int nb, unsigned long long& above, unsigned long long& target,
                              float frac) {
    const int tid = threadIdx.x;
    const int bh = nb - 1 - 2 * tid, bl = bh - 1;
    const unsigned long long vh = bh >= 0 ? sh.bins[bh] : 0ull;
    const unsigned long long vl = bl >= 0 ? sh.bins[bl] : 0ull;
    const unsigned long long val = vh + vl;
    if (tid == 0) {
        sh.pick_bin = 0;
        sh.pick_val = above;
    }
    const unsigned long long incl = block_incl_scan(val, sh.wsum);  // ends with a barrier
    if (frac > 0.f) {
        if (tid == kT - 1) sh.total = incl;  // the level's total
        __syncthreads();
        target = (unsigned long long)((double)frac * (double)sh.total);
    }
    const unsigned long long ex = above + incl - val;  // amount above bin bh
    if (COUNT) {
        if (ex < target && ex + vh >= target) {
            sh.pick_bin = bh;
            sh.pick_val = ex;
        } else if (ex + vh < target && ex + val >= target) {
            sh.pick_bin = bl;
            sh.pick_val = ex + vh;
        }
    } else {
        if (ex <= target && ex + vh > target) {
            sh.pick_bin = bh;
            sh.pick_val = ex;
        } else if (ex + vh <= target && ex + val > target) {
            sh.pick_bin = bl;
            sh.pick_val = ex + vh;
        }
    }
    __syncthreads();
    above = sh.pick_val;
    const uint32_t r = (uint32_t)sh.pick_bin;
    __syncthreads();  // pick_* and the bins are rewritten by the next level
    return r;
}

// The threshold key over register keys >= lo (see above).  l0_binned: the
// first level's bins were filled by the caller (the exponential pass).
template <bool COUNT>
__device__ uint32_t select_key(const uint32_t (&key)[kVPT], uint32_t lo, unsigned long long target, float frac,
                               bool l0_binned, SelShared& sh) {
    unsigned long long above = 0;
    uint32_t b1 = 0, b2 = 0, K = 0;
    bool crowded = false;
#pragma unroll 1
    for (int lv = 0; lv < 3; ++lv) {
        const int shift = lv == 0 ? 19 : (lv == 1 ? 8 : 0);
        const uint32_t mask = lv == 2 ? 255u : 2047u;
        const int pshift = lv == 0 ? 30 : (lv == 1 ? 19 : 8);
        const uint32_t prefix = lv == 0 ? 0u : (lv == 1 ? b1 : ((b1 << 11) | b2));
        if (lv > 0 || !l0_binned) {
            for (int b = threadIdx.x; b < kSelBins; b += kT) sh.bins[b] = 0ull;
            __syncthreads();
            if (lv == 0 || crowded)
                bin_registers<COUNT>(key, lo, shift, mask, pshift, prefix, sh.bins);
            else
                bin_list<COUNT>(sh, shift, mask, pshift, prefix);
            __syncthreads();
        }
        const uint32_t b = scan_pick<COUNT>(sh, (int)mask + 1, above, target, lv == 0 ? frac : 0.f);
        if (lv == 0) {
            b1 = b;
            compact(key, lo, b1, sh);
            __syncthreads();
#pragma unroll
            for (int w = 0; w < kWaves; ++w) crowded |= sh.cnt[w] > kListPerWave;
        } else if (lv == 1) {
            b2 = b;
        } else {
            K = (b1 << 19) | (b2 << 8) | b;
        }
    }
    return K;
}

// Inverse-CDF draw over the kept tokens (key >= lo) in thread-major order with
// u in [0, 1), or (uniform) the fallback for non-finite probabilities: uniform
// over the vocabulary (core.py:102-108).  Writes the row's token and logp.
__device__ __forceinline__ void draw_kept(const uint32_t (&key)[kVPT], uint32_t lo, int V, int rule, bool uniform,
                                          float u, float* fsum, int* pick, SelShared& sh, int64_t* out_tok,
                                          float* out_logp) {
    const int tid = threadIdx.x;
    if (uniform) {
        if (tid == 0) {
            int t = (int)(u * (float)V);
            *out_tok = t < V ? t : V - 1;
            *out_logp = logf(1.0f / (float)V + 1e-10f);
        }
        return;
    }
    float tm = 0.f;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) tm += key[j] >= lo ? __uint_as_float(key[j]) : 0.f;
    if (tid == 0) *pick = -1;
    float before;
    // [before, acc) of consecutive threads tile [0, total) exactly, so exactly one
    // thread with kept mass owns the target (a rounded acc - tm could leave a gap
    // that no thread owns, and the draw unwritten)
    const float acc = block_scan_tiled(tm, fsum, before);
    // every wave reads fsum[0 .. w-1] at the end of the scan: wait for all of
    // them before fsum[0] is reused for the total
    __syncthreads();
    if (tid == kT - 1) fsum[0] = acc;  // the kept mass W
    __syncthreads();
    const float W = fsum[0];
    const float target = u * W;
    if (tm > 0.f && target >= before && (target < acc || acc >= W)) {
        // fully unrolled (no early exit) so key[] stays in registers
        // (the register index is tracked, not the element: elem_of is increasing in
        // it, and 64 element indices would stay live in registers)
        float c = before;
        int chosen = -1;
        bool done = false;
#pragma unroll
        for (int j = 0; j < kVPT; ++j) {
            uint32_t kj = key[j];
            asm volatile("" : "+v"(kj));  // no compare masks kept from the sum above
            const float w = kj >= lo ? __uint_as_float(kj) : 0.f;
            if (!done && w > 0.f) {
                chosen = j;
                c += w;
                done = c > target;
            }
        }
        if (chosen >= 0) atomicMax(pick, elem_of(chosen, tid));
    }
    __syncthreads();
    if (*pick < 0) {
        // not reached when the intervals tile (the total is finite and > 0 here);
        // kept as a deterministic guard: the lowest kept id
        if (tid == 0) sh.pick_bin = 0x7fffffff;
        __syncthreads();
        int first = kVPT;
#pragma unroll
        for (int j = kVPT - 1; j >= 0; --j) {
            uint32_t kj = key[j];
            asm volatile("" : "+v"(kj));
            if (kj >= lo) first = j;
        }
        if (first < kVPT) atomicMin(&sh.pick_bin, elem_of(first, tid));
        __syncthreads();
        if (tid == 0 && sh.pick_bin != 0x7fffffff) *pick = sh.pick_bin;
        __syncthreads();
    }
    const int tok = *pick;
    if (tok >= 0 && tid == owner_of(tok)) {
        uint32_t kq = 0;
#pragma unroll
        for (int j = 0; j < kVPT; ++j)
            if (j == slot_of(tok)) kq = key[j];
        const float q = __uint_as_float(kq);
        *out_tok = tok;
        *out_logp = (rule == RULE_BATCH) ? logf(q) - logf(W) : logf(q / W + 1e-10f);
    }
}

// The two 16-bit logits of a packed word, as floats (low half first).
template <typename LT>
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi);
template <>
__device__ __forceinline__ void unpack2<bf16_t>(uint32_t w, float& lo, float& hi) {
    lo = __uint_as_float(w << 16);
    hi = __uint_as_float(w & 0xffff0000u);
}
template <>
__device__ __forceinline__ void unpack2<f16_t>(uint32_t w, float& lo, float& hi) {
    lo = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
    hi = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// -inf as a 16-bit pattern
template <typename LT> __device__ __forceinline__ uint32_t neg_inf16();
template <> __device__ __forceinline__ uint32_t neg_inf16<bf16_t>() { return 0xff80u; }
template <> __device__ __forceinline__ uint32_t neg_inf16<f16_t>() { return 0xfc00u; }

// A 16-bit row as packed words in the layout of load_row: word 4c + i of thread t
// holds elements 8192 c + 8 t + 2i (low half) and + 1 (high half); entries past
// vmax are -inf.  Same load rules as load_row (no load depends on a condition).
template <typename LT>
__device__ __forceinline__ void load_row16(const LT* lg, int V, int vmax, uint32_t (&w)[kVPT / 2]) {
    const int tid = threadIdx.x;
    if ((((uintptr_t)lg) & 15) == 0 && V % kGroup == 0) {
#pragma unroll
        for (int c = 0; c < kVPT / kGroup; ++c) {
            const int i0 = c * kStride + tid * kGroup;
            const uint4 u = *reinterpret_cast<const uint4*>(lg + (i0 < V ? i0 : 0));
            w[4 * c] = u.x;
            w[4 * c + 1] = u.y;
            w[4 * c + 2] = u.z;
            w[4 * c + 3] = u.w;
        }
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(lg);
#pragma unroll
        for (int c = 0; c < kVPT / kGroup; ++c) {
#pragma unroll
            for (int e = 0; e < kGroup; e += 2) {
                const int i = c * kStride + tid * kGroup + e;
                const uint32_t a = h[i < V ? i : V - 1], b = h[i + 1 < V ? i + 1 : V - 1];
                w[4 * c + e / 2] = a | (b << 16);
            }
        }
    }
    // banned ids and padding (only the threads whose groups reach past vmax)
#pragma unroll
    for (int c = 0; c < kVPT / kGroup; ++c) {
        const int i0 = c * kStride + tid * kGroup;
        if (i0 + kGroup - 1 > vmax) {
#pragma unroll
            for (int e = 0; e < kGroup; e += 2) {
                uint32_t v = w[4 * c + e / 2];
                if (i0 + e > vmax) v = (v & 0xffff0000u) | neg_inf16<LT>();
                if (i0 + e + 1 > vmax) v = (v & 0xffffu) | (neg_inf16<LT>() << 16);
                w[4 * c + e / 2] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Sampled rows of 16-bit logits without logit_bias (the rollout's case).  A
// 16-bit logit takes at most 65,536 values, so the row's histogram over its
// values is an exact sort: one LDS atomic per token builds 65,536 16-bit
// counters (128 KB, two per word), and the rules read the counters in
// descending value order - counts for top-k, mass = count x q(value) in 31-bit
// fixed point (64-bit sums, order-independent) for the nucleus and the draw -
// with one exponential per occupied value instead of one per token.  The draw
// picks a value by an integer inverse CDF over the kept values (every token of a
// value carries the same mass, so this is exact), then the j-th token of that
// value in thread-major order.  Tokens of one value are kept or dropped
// together (ties).  A counter can only overflow when all 65,536 tokens share
// one finite value; the counts then do not add up to V, and the row is drawn
// uniformly over the vocabulary, which is what every rule gives for it.
constexpr int kHist = 65536;

constexpr int kSegs = kHist / 64;  // segments of 64 consecutive value keys

// Greedy rows (temperature < 1e-6, core.py:80-83, 184-188): argmax of the banned
// logits with the lowest index on ties, logp = log_softmax(banned logits)[token].
// Thread t of the 1024-thread block takes elements j * 1024 + t.  Run by
// sample16_kernel for its greedy rows and by greedy_kernel ahead of
// sample_kernel (whose register footprint doubles when it shares a kernel with
// this path).  Not inlined: the sampling path's registers stay its own.
template <typename LT>
__device__ __attribute__((noinline)) void greedy_row(int row, int V, const LT* __restrict__ lg, int max_valid_id,
                                           int64_t* __restrict__ out_tok, float* __restrict__ out_logp, Red* red,
                                           unsigned long long* red64) {
    typedef io_traits<LT> tr;
    const int tid = threadIdx.x;
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
    const float mx = block_max_f(mm, red);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVPTG; ++j) s += (x[j] == -INFINITY) ? 0.f : expf(x[j] - mx);
    const float Z = block_sum_f(s, red);
    if (tid == 0) {
        out_tok[row] = tok;
        // the argmax value is mx unless every logit is -inf / NaN
        out_logp[row] = (mx == -INFINITY) ? -INFINITY : -logf(Z);
    }
}

struct HistShared {
    uint32_t h[kHist / 2];  // counter of value key u: half u & 1 of word u >> 1
    unsigned long long seg_m[kSegs];  // per segment: fixed-point mass and count
    uint32_t seg_c[kSegs];
    unsigned long long wm[kWMax];
    uint32_t wc[kWMax];
    unsigned long long r64[2];
    float rq;
    int r32[5];
};

// order key of a 16-bit float pattern (sign-magnitude to unsigned: larger key,
// larger value) and back
__device__ __forceinline__ uint32_t okey16(uint32_t b) { return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u); }
__device__ __forceinline__ uint32_t bits_of_okey16(uint32_t u) { return (u & 0x8000u) ? (u & 0x7fffu) : (~u & 0xffffu); }

template <typename LT> __device__ __forceinline__ float val16(uint32_t bits);
template <> __device__ __forceinline__ float val16<bf16_t>(uint32_t bits) { return __uint_as_float(bits << 16); }
template <> __device__ __forceinline__ float val16<f16_t>(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
// keys of +inf and -inf: keys above the first and below the second are NaNs
template <typename LT> __device__ __forceinline__ uint32_t key_pinf();
template <> __device__ __forceinline__ uint32_t key_pinf<bf16_t>() { return 0xff80u; }
template <> __device__ __forceinline__ uint32_t key_pinf<f16_t>() { return 0xfc00u; }
template <typename LT> __device__ __forceinline__ uint32_t key_ninf();
template <> __device__ __forceinline__ uint32_t key_ninf<bf16_t>() { return 0x007fu; }
template <> __device__ __forceinline__ uint32_t key_ninf<f16_t>() { return 0x03ffu; }

__device__ __forceinline__ uint32_t hist_count(const HistShared& sh, uint32_t u) {
    return (sh.h[u >> 1] >> ((u & 1u) * 16u)) & 0xffffu;
}

// q of value key u (temperature folded into c1 = log2(e) / T) and its 31-bit
// fixed-point amount: the same expressions wherever a value's mass is needed
template <typename LT>
__device__ __forceinline__ float q_of_key(uint32_t u, float mx, float c1) {
    return fminf(__builtin_amdgcn_exp2f((val16<LT>(bits_of_okey16(u)) - mx) * c1), 1.0f);
}
__device__ __forceinline__ uint32_t fx_of_q(float q) { return (uint32_t)(q * 2147483648.0f); }

// DPP moves (bound_ctrl: lanes whose source lies outside the row read 0)
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long x) {
    const uint32_t lo = dpp_u32<CTRL>((uint32_t)x), hi = dpp_u32<CTRL>((uint32_t)(x >> 32));
    return ((unsigned long long)hi << 32) | lo;
}
// sum over the 16 lanes of a row, in every lane of it (row_mirror, row_half_mirror,
// then quad permutations: each step adds a disjoint partner set)
template <typename T>
__device__ __forceinline__ T row_sum16(T x) {
    if constexpr (sizeof(T) == 8) {
        x += dpp_u64<0x140>(x);
        x += dpp_u64<0x141>(x);
        x += dpp_u64<0x4e>(x);
        x += dpp_u64<0xb1>(x);
    } else {
        x += dpp_u32<0x140>(x);
        x += dpp_u32<0x141>(x);
        x += dpp_u32<0x4e>(x);
        x += dpp_u32<0xb1>(x);
    }
    return x;
}
// maximum over the 64 lanes (NaNs ignored, as fmaxf does), in every lane: row
// maxima by the row_sum16 partner pattern, then the four rows' from lanes 0, 16,
// 32, 48
__device__ __forceinline__ float wave_max16(float x) {
    x = fmaxf(x, __builtin_amdgcn_update_dpp(x, x, 0x140, 0xf, 0xf, false));
    x = fmaxf(x, __builtin_amdgcn_update_dpp(x, x, 0x141, 0xf, 0xf, false));
    x = fmaxf(x, __builtin_amdgcn_update_dpp(x, x, 0x4e, 0xf, 0xf, false));
    x = fmaxf(x, __builtin_amdgcn_update_dpp(x, x, 0xb1, 0xf, 0xf, false));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// inclusive scan over the 64 lanes in lane order: row scans by row_shr 1, 2, 4, 8,
// then the totals of the rows below (read from lanes 15, 31, 47)
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T x) {
    if constexpr (sizeof(T) == 8) {
        x += dpp_u64<0x111>(x);
        x += dpp_u64<0x112>(x);
        x += dpp_u64<0x114>(x);
        x += dpp_u64<0x118>(x);
    } else {
        x += dpp_u32<0x111>(x);
        x += dpp_u32<0x112>(x);
        x += dpp_u32<0x114>(x);
        x += dpp_u32<0x118>(x);
    }
    T r[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        if constexpr (sizeof(T) == 8) {
            const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)x, 16 * i + 15);
            const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), 16 * i + 15);
            r[i] = ((unsigned long long)hi << 32) | lo;
        } else {
            r[i] = (T)__builtin_amdgcn_readlane((int)x, 16 * i + 15);
        }
    }
    const int row = (threadIdx.x & 63) >> 4;
    return x + (row > 0 ? r[0] : T(0)) + (row > 1 ? r[1] : T(0)) + (row > 2 ? r[2] : T(0));
}

// Inclusive scan in thread order of (count, fixed-point mass), with the totals.
__device__ __forceinline__ void block_scan2(uint32_t& c, unsigned long long& m, HistShared& sh, uint32_t& tc,
                                            unsigned long long& tm) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    c = wave_incl_scan(c);
    m = wave_incl_scan(m);
    if (lane == 63) {
        sh.wc[w] = c;
        sh.wm[w] = m;
    }
    __syncthreads();
    uint32_t oc = 0;
    unsigned long long om = 0;
    tc = 0;
    tm = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        if (i < w) {
            oc += sh.wc[i];
            om += sh.wm[i];
        }
        tc += sh.wc[i];
        tm += sh.wm[i];
    }
    c += oc;
    m += om;
}

// exclusive scan of a count in thread order (the caller makes sure no thread still
// reads wc: in sample16_kernel at least two barriers separate it from block_scan2)
__device__ __forceinline__ uint32_t block_excl_scan_u32(uint32_t v, HistShared& sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t x = wave_incl_scan(v);
    if (lane == 63) sh.wc[w] = x;
    __syncthreads();
    uint32_t off = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i)
        if (i < w) off += sh.wc[i];
    return x - v + off;
}

// Walk of one segment by wave 0, lane j on key 64 seg + 63 - j (descending),
// from the amounts above the segment (r32[0] count, r64[0] mass; segment in
// r32[1]): finds the first key where the running count reaches `target` (COUNT)
// or the running fixed-point mass exceeds it, and publishes it: r32[2] = key,
// r32[3] = its count, r32[4] = its amount per token, rq = its q, r64[1] = the
// mass above it.  Called by every thread (barriers inside); the segment holds
// the target, so a key is found.
template <typename LT, bool COUNT>
__device__ __forceinline__ void walk_segment(HistShared& sh, unsigned long long target, float mx, float c1) {
    __syncthreads();  // the caller's r* writes
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const uint32_t seg = (uint32_t)sh.r32[1];
        const uint32_t u = 64u * seg + 63u - (uint32_t)lane;
        const uint32_t n = hist_count(sh, u);
        float q = 0.f;
        uint32_t a = 0u;
        if (n != 0u) {
            q = q_of_key<LT>(u, mx, c1);
            a = fx_of_q(q);
        }
        const unsigned long long mine = (unsigned long long)n * a;
        bool hit;
        unsigned long long m = 0ull;
        if (COUNT) {
            const uint32_t c = wave_incl_scan(n);
            hit = (unsigned long long)(uint32_t)sh.r32[0] + c >= target;
            m = wave_incl_scan(mine);
        } else {
            m = wave_incl_scan(mine);
            hit = sh.r64[0] + m > target;
        }
        const unsigned long long hits = __ballot(hit);
        if (hits != 0ull && lane == __builtin_ctzll(hits)) {
            sh.r32[2] = (int)u;
            sh.r32[3] = (int)n;
            sh.r32[4] = (int)a;
            sh.rq = q;
            sh.r64[1] = sh.r64[0] + m - mine;
        }
    }
    __syncthreads();
}

template <typename LT>
__global__ __launch_bounds__(kT) void sample16_kernel(
    int M, int V, const LT* __restrict__ logits, int64_t ld, int rule, int max_valid_id,
    const float* __restrict__ temperature, const float* __restrict__ top_p,
    const int32_t* __restrict__ top_k, const uint8_t* __restrict__ active, uint64_t seed,
    const int64_t* __restrict__ rng_key, const int32_t* __restrict__ rng_ctr, int64_t* __restrict__ out_tok,
    float* __restrict__ out_logp)
{
    __shared__ Red red;
    __shared__ HistShared sh;
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;  // whole block
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float temp = temperature[row];
    if (!(temp >= 1e-6f)) {  // greedy row (the counters' words serve as its reduction space)
        greedy_row<LT>(row, V, logits + (size_t)row * ld, max_valid_id, out_tok, out_logp, &red, sh.wm);
        return;
    }
    const int vmax = max_valid_id < V - 1 ? max_valid_id : V - 1;
    uint32_t w[kVPT / 2];
    load_row16<LT>(logits + (size_t)row * ld, V, vmax, w);
    {   // clear the counters (ordered before the atomics by the barrier of the maximum)
        uint4* hz = reinterpret_cast<uint4*>(sh.h);
#pragma unroll
        for (int i = 0; i < kHist / 2 / 4 / kT; ++i) hz[i * kT + tid] = make_uint4(0u, 0u, 0u, 0u);
    }
    float mm = -INFINITY;
#pragma unroll
    for (int i = 0; i < kVPT / 2; ++i) {
        float a, b;
        unpack2<LT>(w[i], a, b);
        mm = fmaxf(mm, fmaxf(a, b));
    }
    // row maximum (NaNs do not count here; their keys are found below); the
    // barrier also orders the clearing of the counters before the atomics
    mm = wave_max16(mm);
    if (lane == 0) red.f[wv] = mm;
    __syncthreads();
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) mx = fmaxf(mx, red.f[i]);
#pragma unroll
    for (int i = 0; i < kVPT / 2; ++i) {
        const uint32_t ua = okey16(w[i] & 0xffffu), ub = okey16(w[i] >> 16);
        atomicAdd(&sh.h[ua >> 1], 1u << ((ua & 1u) * 16u));
        atomicAdd(&sh.h[ub >> 1], 1u << ((ub & 1u) * 16u));
    }
    __syncthreads();

    // per-segment totals: segment 4 (16 i + wave) + row is summed by a row of 16
    // lanes of the wave (four segments per wave and step, 16 steps), four keys per
    // lane; a step whose four segments are empty writes zeros and skips the rest.
    // q = exp((l - max) / T) = exp2((l - max) * log2(e) / T), with the reciprocal
    // temperature (within an ulp of the division); the maximum gets exactly 1
    const float c1 = (temp != 1.0f ? 1.0f / temp : 1.0f) * 1.4426950408889634f;
    const uint32_t kpinf = key_pinf<LT>(), kninf = key_ninf<LT>();
    const int my_seg = kSegs - 1 - tid;
    bool nan = false;
    {
        const int r = lane & 15;
#pragma unroll 1
        for (int i = 0; i < kSegs / (4 * kWaves); ++i) {
            const uint32_t seg = (uint32_t)(4 * (kWaves * i + wv) + (lane >> 4));
            // this lane's keys 64 seg + 4 r .. + 3: words 32 seg + 2 r, + 1
            const uint2 wd = *reinterpret_cast<const uint2*>(&sh.h[32 * seg + 2 * r]);
            uint32_t c = 0u;
            unsigned long long m = 0ull;
            if (__ballot((wd.x | wd.y) != 0u) != 0ull) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t n = ((e < 2 ? wd.x : wd.y) >> ((e & 1) * 16)) & 0xffffu;
                    if (n != 0u) {
                        const uint32_t u = 64u * seg + 4u * (uint32_t)r + (uint32_t)e;
                        if (u > kpinf || u < kninf) {
                            nan = true;
                        } else {
                            c += n;
                            m += (unsigned long long)n * fx_of_q(q_of_key<LT>(u, mx, c1));
                        }
                    }
                }
                c = row_sum16(c);
                m = row_sum16(m);
            }
            if (r == 0) {
                sh.seg_c[seg] = c;
                sh.seg_m[seg] = m;
            }
        }
    }
    const bool any_nan = __syncthreads_or(nan);
    const uint32_t own_c = sh.seg_c[my_seg];
    const unsigned long long own_m = sh.seg_m[my_seg];
    uint32_t inc_c = own_c, tc;
    unsigned long long inc_m = own_m, tmx;
    block_scan2(inc_c, inc_m, sh, tc, tmx);
    const uint32_t exc_c = inc_c - own_c;
    const unsigned long long exc_m = inc_m - own_m;
    const float u01 = uniform01(seed, (uint64_t)rng_key[row], (uint64_t)(uint32_t)rng_ctr[row]);
    // (with a finite maximum the sum of q lies in [1, 65536]: only NaNs and
    // infinite maxima make the probabilities non-finite)
    const bool uniform = any_nan || !(mx > -INFINITY) || !(mx < INFINITY);
    if (uniform || tc != (uint32_t)(kT * kVPT)) {  // every register slot was counted, padding included
        // non-finite probabilities: uniform over the vocabulary (core.py:102-108);
        // otherwise all 65,536 entries share one finite value (a counter
        // overflowed: V = 65,536, no ban) and every rule keeps them all: uniform,
        // q = 1, W = V
        if (tid == 0) {
            int t = (int)(u01 * (float)V);
            out_tok[row] = t < V ? t : V - 1;
            out_logp[row] = (!uniform && rule == RULE_BATCH) ? -logf((float)V) : logf(1.0f / (float)V + 1e-10f);
        }
        return;
    }

    // kept: keys >= K, a prefix of the descending keys, with fixed-point mass Wfx
    const int k = top_k[row];
    const float p = top_p[row];
    const bool topk = k > 0 && k < V;
    const bool nucleus = p < 1.0f && (rule == RULE_BATCH || (rule == RULE_MIXIN && p > 0.f) ||
                                      (rule == RULE_SINGLE && k <= 0));
    unsigned long long Wfx = tmx;
    if (topk) {
        // the k-th largest value: the running count (over every entry) first reaches k
        const unsigned long long kk = (unsigned long long)k;
        if (exc_c < kk && (unsigned long long)inc_c >= kk) {
            sh.r32[0] = (int)exc_c;
            sh.r32[1] = my_seg;
            sh.r64[0] = exc_m;
        }
        walk_segment<LT, true>(sh, kk, mx, c1);
        // (a walk's inputs and results are disjoint slots, and the next walk writes
        // its results only after its first barrier: no barrier needed after this read)
        Wfx = sh.r64[1] + (unsigned long long)(uint32_t)sh.r32[3] * (uint32_t)sh.r32[4];
    }
    if (nucleus) {
        // the value whose inclusion crosses p of the kept mass: the running mass
        // first exceeds floor(p * Wfx)
        const unsigned long long target = (unsigned long long)((double)fmaxf(p, 1e-30f) * (double)Wfx);
        if (exc_m <= target && inc_m > target) {
            sh.r32[0] = (int)exc_c;
            sh.r32[1] = my_seg;
            sh.r64[0] = exc_m;
        }
        walk_segment<LT, false>(sh, target, mx, c1);
        // RULE_SINGLE / RULE_MIXIN keep the crossing value; RULE_BATCH stops
        // before it but always keeps the most probable value
        const unsigned long long above = sh.r64[1];
        const bool keep = rule != RULE_BATCH || above == 0ull;
        Wfx = keep ? above + (unsigned long long)(uint32_t)sh.r32[3] * (uint32_t)sh.r32[4] : above;
    }

    // the draw: a value by the integer inverse CDF over the kept prefix (target <
    // Wfx), then the j-th token of that value
    const unsigned long long td = (unsigned long long)((double)u01 * (double)Wfx);
    if (exc_m <= td && inc_m > td) {
        sh.r32[0] = (int)exc_c;
        sh.r32[1] = my_seg;
        sh.r64[0] = exc_m;
    }
    walk_segment<LT, false>(sh, td, mx, c1);
    const uint32_t vb = bits_of_okey16((uint32_t)sh.r32[2]);
    const uint32_t jth = (uint32_t)((td - sh.r64[1]) / (uint32_t)sh.r32[4]);  // amount > 0: the value holds td
    const float qd = sh.rq;
    uint32_t oc = 0;
#pragma unroll
    for (int i = 0; i < kVPT / 2; ++i) {
        uint32_t x = w[i];
        asm volatile("" : "+v"(x));
        oc += ((x & 0xffffu) == vb) + ((x >> 16) == vb);
    }
    const uint32_t exc_o = block_excl_scan_u32(oc, sh);
    if (jth >= exc_o && jth < exc_o + oc) {
        int r = (int)(jth - exc_o), jr = -1;
#pragma unroll
        for (int i = 0; i < kVPT / 2; ++i) {
            uint32_t x = w[i];
            asm volatile("" : "+v"(x));
            if ((x & 0xffffu) == vb) {
                if (r == 0) jr = 2 * i;
                --r;
            }
            if ((x >> 16) == vb) {
                if (r == 0) jr = 2 * i + 1;
                --r;
            }
        }
        // the kept mass W = Wfx / 2^31: each kept token's amount is q 2^31 truncated,
        // so this is within (kept tokens) / 2^31 of the float sum
        const float W = (float)Wfx * 4.656612873077393e-10f;
        out_tok[row] = elem_of(jr, tid);
        out_logp[row] = (rule == RULE_BATCH) ? logf(qd) - logf(W) : logf(qd / W + 1e-10f);
    }
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
    __shared__ SelShared sh;
    __shared__ float fsum[kWMax];
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

    const int k = top_k[row];
    const float p = top_p[row];
    const bool topk = k > 0 && k < V;
    const bool nucleus = p < 1.0f && (rule == RULE_BATCH || (rule == RULE_MIXIN && p > 0.f) ||
                                      (rule == RULE_SINGLE && k <= 0));
    // with no top-k before it, the nucleus's first level is binned in the exponential pass
    const bool fused = nucleus && !topk;
    if (fused)
        for (int b = tid; b < kSelBins; b += kT) sh.bins[b] = 0ull;  // ordered by the reductions' barriers

    float mm = -INFINITY;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) mm = fmaxf(mm, x[j]);
    const float mx = block_max_f(mm, &red);
    // From here on a token is its key: the bit pattern of q = exp(l - max) >= 0
    // (0 for banned and padding entries), which orders like the logit; q is read
    // back by reinterpreting the key, and one register per token keeps the row.
    // A NaN logit stays NaN here (the compare is false), so Z turns NaN and the
    // row takes the uniform fallback, as the reference's isnan(probs) does.
    uint32_t key[kVPT];
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kVPT; ++j) {
        const float e = fast_exp(x[j] - mx);
        const float q = (x[j] == -INFINITY) ? 0.f : (e > 1.0f ? 1.0f : e);
        key[j] = __float_as_uint(q);
        s += q;
        // first level of the nucleus (keys >= 1, bits 19..29)
        if (fused && key[j] != 0u) atomicAdd(&sh.bins[(key[j] >> 19) & 2047u], sel_amount<false>(key[j]));
    }
    const float Z = block_sum_f(s, &red);
    const bool uniform = !(mx > -INFINITY) || !(mx < INFINITY) || !(Z < INFINITY) || !(Z > 0.f);

    // kept set: key >= lo (lo = 1: every token with non-zero probability)
    uint32_t lo = 1;
    if (!uniform && topk) {
        // the k-th largest key: the highest K with count(key >= K) >= k (over every
        // token, so that k < V always has an answer)
        const uint32_t K = select_key<true>(key, 0u, (unsigned long long)k, 0.f, false, sh);
        lo = K > 1u ? K : 1u;
    }
    if (!uniform && nucleus) {
        // the key of the token whose inclusion crosses p: the highest K' with
        // mass(key >= max(K', lo)) > p * mass(key >= lo), in fixed point
        const uint32_t K = select_key<false>(key, lo, 0ull, fmaxf(p, 1e-30f), fused, sh);
        // RULE_SINGLE and RULE_MIXIN keep the crossing token, RULE_BATCH stops
        // before it but always keeps the most probable token (q = 1)
        uint32_t nlo = (rule == RULE_BATCH) ? K + 1u : K;
        const uint32_t top = __float_as_uint(1.0f);
        if (nlo > top) nlo = top;
        lo = nlo > lo ? nlo : lo;
    }

    draw_kept(key, lo, V, rule, uniform, uniform01(seed, (uint64_t)rng_key[row], (uint64_t)(uint32_t)rng_ctr[row]),
              fsum, &pick, sh, out_tok + row, out_logp + row);
}

template <typename LT>
__global__ __launch_bounds__(kTG) void greedy_kernel(
    int M, int V, const LT* __restrict__ logits, int64_t ld, int max_valid_id,
    const float* __restrict__ temperature, const uint8_t* __restrict__ active,
    int64_t* __restrict__ out_tok, float* __restrict__ out_logp)
{
    __shared__ Red red;
    __shared__ unsigned long long red64[kWMax];
    const int row = blockIdx.x;
    if (active != nullptr && active[row] == 0) return;
    if (temperature[row] >= 1e-6f) return;  // sampled rows belong to sample_kernel
    greedy_row<LT>(row, V, logits + (size_t)row * ld, max_valid_id, out_tok, out_logp, &red, red64);
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
    if constexpr (sizeof(LT) == 2) {
        if (bias_off == nullptr) {  // one launch: sample16_kernel takes the greedy rows too
            hipLaunchKernelGGL(sample16_kernel<LT>, dim3(M), dim3(kT), 0, st, M, V, (const LT*)logits, ld, rule,
                               max_valid_id, temperature, top_p, top_k, active, seed, rng_key, rng_ctr, out_tok,
                               out_logp);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL(greedy_kernel<LT>, dim3(M), dim3(kTG), 0, st, M, V, (const LT*)logits, ld, max_valid_id,
                       temperature, active, out_tok, out_logp);
    const hipError_t e = hipGetLastError();
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
