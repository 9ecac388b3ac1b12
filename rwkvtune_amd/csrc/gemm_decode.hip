// Grouped bf16 GEMM for the decode step's projections on gfx950 MFMA.
//
// At decode the model's dense projections have M = live slots (<= 256) rows:
// r / k / v / output (C x C), the LoRA downs (C x 64..480), the FFN
// (C x 4C, 4C x C) and the head (C x V).  One launch runs up to 8 independent
// problems
//     C_p[M, N_p] = epi_p( A_p[M, K_p] . B_p[N_p, K_p]^T )
// with A row-major, B an nn.Linear weight [out][in] (N x K) stored in the
// packed layout below, bf16 in, fp32 accumulate, bf16 out.  epi: 0 none,
// 1 relu(x)^2 (FFN key, model.py:337), 2 tanh, 3 sigmoid (the LoRA activations
// of model.py:211, 221, applied to a down projection's output).
//
// At M <= 256 every weight byte is used by at most 256 rows, so a projection
// is bound by streaming its weights (close to the MFMA / HBM ridge at M = 256,
// far below it for fewer rows).  The kernel is built for that:
//   * weights are packed once (gemm_pack_kernel) into 64 x 64 tiles, each a
//     contiguous 8 KB block already in the block's LDS order, tiles of one
//     64-row group consecutive along K: a stage's weight load is one linear
//     8 KB copy.  Read in place, an [out][in] matrix gives 64 separate 128-byte
//     segments per stage, and HBM streams such a pattern at ~1.7 TB/s against
//     ~5 TB/s for long contiguous runs (measured on MI355X);
//   * a block of 4 or 8 waves computes a BM x BN tile (a template: waves in a
//     WM x WN grid, each MS x NS tiles of v_mfma_f32_32x32x16_bf16; BN a
//     multiple of 32); the tile and the K split are chosen by row count.  A CU moves roughly 30-40 GB/s of vector loads whether
//     they hit L2 or not (measured), so at M = 256 the activation re-reads,
//     not the weights, dominate a small tile; large tiles cut them, and split
//     K restores the block count;
//   * K advances 64 at a time through a ring of R LDS stages filled by direct
//     global -> LDS loads (global_load_lds_dwordx4: no registers, no LDS store
//     instructions), R - 1 stages in flight.  Each stage costs one barrier; the
//     wait before it names its own count of outstanding loads (s_waitcnt
//     vmcnt(n)), so the loads of later stages stay in flight;
//   * weight loads carry the non-temporal hint: a decode step streams every
//     layer's weights once (2.4 GB at 1.5B, far beyond L2 and the last-level
//     cache), and the hint keeps them from displacing the activation rows every
//     column tile re-reads (cfg4 rollout decode 2.353 -> 2.306 s, same box);
//   * a stage row is 64 bf16 = 8 chunks of 16 bytes; chunk c of stage row r
//     sits at position c ^ swz(r), which keeps the MFMA operand reads (32 rows,
//     one chunk each) free of LDS bank conflicts;
//   * A chunks past a problem's K read a 16-byte zero page instead (direct
//     loads cannot be masked; packed weights are zero-padded to whole tiles),
//     rows past M read a valid row whose results are not stored;
//   * blocks are ordered so that the row tiles and K ranges of one column tile
//     run back to back on one XCD (blocks are dealt to the 8 XCDs round-robin),
//     where they share the weight rows through that XCD's L2;
//   * problems with too few tiles to fill the GPU split K; each range writes
//     float32 partial rows to the caller's workspace and gemm_reduce_kernel sums
//     the ranges in order (deterministic) and applies the epilogue - or, for
//     launch_gemm_decode_partials, the consumer of the result does.
// MFMA operand layout (gfx950): lane l supplies row l%32 of A and of B, k =
// 8*(l/32) .. +7; accumulator q of lane l is C[8*(q/4) + 4*(l/32) + q%4][l%32].
#include <mutex>

#include "common.hpp"
#include "rwkv7_hip.h"

// source of the chunks past a K range
__device__ __attribute__((aligned(16))) uint32_t g_gemm_zero_chunk[4];

// Split-K partials of rwkv7_gemm_decode_noalloc: a fixed array in every GPU's
// copy of the code object (RWKV7_GEMM_SCRATCH_FLOATS floats, held until the
// process ends), used instead of a caller workspace.  Host code never passes
// the array's name to a kernel: that is a host-side stand-in, not a device
// address.  gemm_scratch() looks up each device's address once, with
// hipGetSymbolAddress on that device, and every launch takes the looked-up pointer.
static __device__ __align__(256) float scratch[RWKV7_GEMM_SCRATCH_FLOATS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// Device address of the current device's scratch array (looked up on the first
// call on that device).
hipError_t gemm_scratch(float** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxProblems = 8;
constexpr int BK = 64;                 // k per stage: one 128-byte row segment

struct GemmProblem {
    const bf16_t* A;
    const bf16_t* B;  // packed
    bf16_t* C;
    int64_t lda, ldc;
    int64_t ws_off;   // float offset of this problem's partials in the workspace
    int N, K;
    int epi;
    int block_begin;  // first block of this problem (a multiple of 8)
    int n_tiles;      // tiles along N
    int k_tiles;      // 64-wide K tiles of the packed weight
    int n64;          // 64-row tiles of the packed weight
    int splits;       // K ranges
    int k_per;        // K per range (multiple of BK)
    int red_begin;    // first block of this problem in gemm_reduce_kernel
    int partial;      // 1: write float32 partials even when splits == 1 (no epilogue)
};

struct GemmBatch {
    GemmProblem p[kMaxProblems];
    int count;
    int M;
    int bm, bn;       // tile of the launch
};

// Block tile: WM x WN x KG waves, each wave MS x NS MFMA tiles of 32 x 32 over
// 1/KG of each stage's K steps (KG wave groups, summed at the end); a ring of
// R LDS stages.  More waves per block means more waves issuing loads: one
// wave's direct loads stream at ~35 GB/s (measured), a CU's at ~130 GB/s.
template <int WM_, int WN_, int MS_, int NS_, int R_, int KG_ = 1>
struct Tile {
    static constexpr int WM = WM_, WN = WN_, MS = MS_, NS = NS_, R = R_, KG = KG_;
    static constexpr int NWAVE = WM * WN * KG, THREADS = 64 * NWAVE;
    static constexpr int BM = 32 * MS * WM, BN = 32 * NS * WN;
    static constexpr int ROWS = BM + BN;          // stage rows: A rows, then B rows
    static constexpr int IPW = ROWS / 8 / NWAVE;  // direct loads per wave per stage (8 rows each)
    static constexpr int STAGE = ROWS * 128;      // bytes
    static_assert(NWAVE == 4 || NWAVE == 8 || NWAVE == 16, "4, 8 or 16 waves per block");
    static_assert(KG == 1 || KG == 2 || KG == 4, "K-step groups divide the 4 steps of a stage");
    static_assert(BN % 32 == 0, "column tiles of 32 or whole 64-row packed tiles");
    static_assert(IPW * 8 * NWAVE == ROWS, "loads split evenly over the waves");
    static_assert(R >= 2 && (R - 2) * IPW < 64, "vmcnt holds at most 63 outstanding loads");
    static_assert(R * STAGE <= 160 * 1024, "LDS");
};

// LDS position of logical chunk c in stage row r (conflict-free for 32 and 64 banks)
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }

// s_waitcnt vmcnt(N) lgkmcnt(0)
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

__device__ __forceinline__ float epi_fn(int epi, float v) {
    if (epi == 1) {
        v = v > 0.f ? v : 0.f;
        return v * v;
    }
    if (epi == 2) return tanhf(v);
    if (epi == 3) return 1.0f / (1.0f + expf(-v));
    return v;
}

__device__ __forceinline__ GemmProblem select_problem(const GemmBatch& batch, int bid, bool reduce) {
    // constant indices only: a dynamic index into the kernel-argument struct
    // would copy it to scratch memory
    GemmProblem P = batch.p[0];
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < batch.count && bid >= (reduce ? batch.p[i].red_begin : batch.p[i].block_begin)) P = batch.p[i];
    return P;
}

// Issue stage s's direct loads into its ring slot.  An A load whose 8 rows all
// lie past the last real row reads the zero page (an L2 hit): those rows feed
// only outputs that are never stored.  Every wave issues IPW loads per stage,
// which the kernel's waits count on.  (A device function rather than a lambda
// in the kernel: with a non-zero cache hint in a lambda the host pass drops
// the kernel's launch stub.)
template <class T>
__device__ __forceinline__ void issue_stage(uint8_t* ring, const bf16_t* const (&src)[T::IPW], const int (&kc)[T::IPW],
                                            int s, int wave, int m0, int M, int kspan, const bf16_t* zero) {
    uint8_t* dst = ring + (s % T::R) * T::STAGE;
#pragma unroll
    for (int i = 0; i < T::IPW; ++i) {
        const int row0 = 8 * (i * T::NWAVE + wave);  // wave-uniform
        if (row0 >= T::BM) {
            // weights: non-temporal (aux 2), they are read once per step
            __builtin_amdgcn_global_load_lds(src[i] + s * (64 * BK), dst + row0 * 128, 16, 0, 2);
        } else {
            const bf16_t* g = (m0 + row0 < M && s * BK + kc[i] < kspan) ? src[i] + s * BK : zero;
            __builtin_amdgcn_global_load_lds(g, dst + row0 * 128, 16, 0, 0);
        }
    }
}

template <class T>
__global__ __launch_bounds__(T::THREADS) void gemm_decode_kernel(GemmBatch batch, float* __restrict__ ws) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[T::R * T::STAGE];

    const GemmProblem P = select_problem(batch, blockIdx.x, false);
    const int M = batch.M;
    const int mt = (M + T::BM - 1) / T::BM;
    const int local = blockIdx.x - P.block_begin;
    const int xcd = local & 7, j = local >> 3;  // block_begin is a multiple of 8: same XCD as blockIdx.x
    const int per = mt * P.splits;
    const int ntile = (j / per) * 8 + xcd;
    if (ntile >= P.n_tiles) return;             // padding block of the last column group
    const int rem = j % per;
    const int mtile = rem % mt, split = rem / mt;
    const int m0 = mtile * T::BM, n0 = ntile * T::BN;
    const int kb = split * P.k_per;
    const int kspan = min(P.K, kb + P.k_per) - kb;
    const int nst = (kspan + BK - 1) / BK;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Direct loads: load i of wave w fills stage rows 8 (i NWAVE + w) .. +7, A rows
    // first, so the activation and the weight loads are spread over all the
    // waves (with BM = BN every wave issues one of each per stage, which streams
    // ~10% faster than giving the two halves to separate waves).  For an A row,
    // lane L brings logical chunk (L%8) ^ swz(row) of row 8 (i NWAVE + w) + L/8 to
    // LDS position L%8 of that row; a B load is a linear 1 KB piece of the packed
    // tile, which holds the same arrangement.
    const bf16_t* src[T::IPW];
    int kc[T::IPW];  // k offset of the lane's A chunk within a stage (-1: B load)
    const int kt0 = kb / BK;
#pragma unroll
    for (int i = 0; i < T::IPW; ++i) {
        const int row0 = 8 * (i * T::NWAVE + wave);
        if (row0 < T::BM) {
            const int row = row0 + (lane >> 3);
            const int c = (lane & 7) ^ swz(row);
            kc[i] = 8 * c;
            src[i] = P.A + (int64_t)min(m0 + row, M - 1) * P.lda + kb + 8 * c;
        } else {
            // weight rows n0 + rr0 .. +7 lie in one 64-row packed tile; tiles past
            // the weight (N not a multiple of BN) re-read its last tile
            const int wr0 = n0 + row0 - T::BM;
            const int t64 = min(wr0 / 64, P.n64 - 1);
            kc[i] = -1;
            src[i] = P.B + ((int64_t)t64 * P.k_tiles + kt0) * (64 * BK) + (wr0 % 64) * BK + lane * 8;
        }
    }
    const bf16_t* zero = reinterpret_cast<const bf16_t*>(g_gemm_zero_chunk);

    f32x16 acc[T::MS][T::NS];
#pragma unroll
    for (int a = 0; a < T::MS; ++a)
#pragma unroll
        for (int b = 0; b < T::NS; ++b) acc[a][b] = f32x16{0.f};
    const int lr = lane & 31, hi = lane >> 5;
    const int wt = wave % (T::WM * T::WN), kgrp = wave / (T::WM * T::WN);
    const int wm = (wt / T::WN) * (32 * T::MS), wn = (wt % T::WN) * (32 * T::NS);
    constexpr int KS = 4 / T::KG;  // k steps of 16 per stage for this wave
    auto mma = [&](int s) {
        const uint8_t* st = ring + (s % T::R) * T::STAGE;
        // every operand of the stage is read before the first product, so the
        // LDS latency is paid once per stage rather than once per k step
        bf16x8_t af[KS][T::MS], bfr[KS][T::NS];
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            const int c = 2 * (kgrp * KS + kk) + hi;
#pragma unroll
            for (int a = 0; a < T::MS; ++a) {
                const int row = wm + 32 * a + lr;
                af[kk][a] = *reinterpret_cast<const bf16x8_t*>(st + row * 128 + ((c ^ swz(row)) << 4));
            }
#pragma unroll
            for (int b = 0; b < T::NS; ++b) {
                // row of the B part; its chunks are swizzled by its row in the packed tile
                const int row = wn + 32 * b + lr;
                bfr[kk][b] = *reinterpret_cast<const bf16x8_t*>(st + (T::BM + row) * 128 +
                                                                 ((c ^ swz((n0 + row) & 63)) << 4));
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the products
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int a = 0; a < T::MS; ++a)
#pragma unroll
                for (int b = 0; b < T::NS; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk][a], bfr[kk][b], acc[a][b], 0, 0, 0);
    };

    // Stage s lives in slot s % R.  Iteration s: wait until this wave's loads of
    // stage s have landed (the R - 2 later stages may still be in flight) and
    // its LDS reads of stage s - 1 are done; the barrier then makes every
    // wave's share of stage s visible, and tells every wave that slot
    // (s - 1) % R is no longer read, so stage s + R - 1 is issued into it.
#pragma unroll
    for (int s = 0; s < T::R - 1; ++s)
        if (s < nst) issue_stage<T>(ring, src, kc, s, wave, m0, M, kspan, zero);
    for (int s = 0; s < nst; ++s) {
        if (s + T::R - 2 < nst)
            wait_vm_lgkm<(T::R - 2) * T::IPW>();
        else
            wait_vm_lgkm<0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS read moves above the barrier
        if (s + T::R - 1 < nst) issue_stage<T>(ring, src, kc, s + T::R - 1, wave, m0, M, kspan, zero);
        mma(s);
    }

    if constexpr (T::KG > 1) {
        // sum the K groups' accumulators into group 0 through the (now idle) ring
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        float* red = reinterpret_cast<float*>(ring);
        constexpr int PER = T::MS * T::NS * 16;  // floats per lane
        static_assert((size_t)(T::KG - 1) * T::WM * T::WN * 64 * PER * 4 <= (size_t)T::R * T::STAGE, "LDS");
        if (kgrp > 0) {
            float* dst = red + ((size_t)((kgrp - 1) * T::WM * T::WN + wt) * PER) * 64 + lane;
#pragma unroll
            for (int a = 0; a < T::MS; ++a)
#pragma unroll
                for (int b = 0; b < T::NS; ++b)
#pragma unroll
                    for (int q = 0; q < 16; ++q) dst[((a * T::NS + b) * 16 + q) * 64] = acc[a][b][q];
        }
        __syncthreads();
        if (kgrp > 0) return;
#pragma unroll
        for (int g = 1; g < T::KG; ++g) {
            const float* srcp = red + ((size_t)((g - 1) * T::WM * T::WN + wt) * PER) * 64 + lane;
#pragma unroll
            for (int a = 0; a < T::MS; ++a)
#pragma unroll
                for (int b = 0; b < T::NS; ++b)
#pragma unroll
                    for (int q = 0; q < 16; ++q) acc[a][b][q] += srcp[((a * T::NS + b) * 16 + q) * 64];
        }
    }

    if (P.splits == 1 && !P.partial) {
#pragma unroll
        for (int a = 0; a < T::MS; ++a)
#pragma unroll
            for (int b = 0; b < T::NS; ++b) {
                const int col = n0 + wn + 32 * b + lr;
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int row = m0 + wm + 32 * a + 8 * (q >> 2) + 4 * hi + (q & 3);
                    if (row < M && col < P.N)
                        P.C[(int64_t)row * P.ldc + col] = f32_to_bf16(epi_fn(P.epi, acc[a][b][q]));
                }
            }
        return;
    }
    // split-K: publish this range's partial products as rows of the float32
    // [splits][M][N] array at the problem's workspace offset; gemm_reduce_kernel,
    // launched next on the same stream, or the consumer of the partials sums
    // the ranges in order (a kernel boundary is what makes another block's
    // writes visible: the L2 of each XCD is private)
    float* part = ws + P.ws_off + (int64_t)split * M * P.N;
#pragma unroll
    for (int a = 0; a < T::MS; ++a)
#pragma unroll
        for (int b = 0; b < T::NS; ++b) {
            const int col = n0 + wn + 32 * b + lr;
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int row = m0 + wm + 32 * a + 8 * (q >> 2) + 4 * hi + (q & 3);
                if (row < M && col < P.N) part[(int64_t)row * P.N + col] = acc[a][b][q];
            }
        }
}

// Sum the split-K partials in split order (deterministic), apply the epilogue
// and write bf16.  Thread e of problem p covers 4 consecutive elements of the
// problem's [M][N] partial rows; red_begin is the problem's first block here.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmBatch batch, const float* __restrict__ ws) {
    const GemmProblem P = select_problem(batch, blockIdx.x, true);
    const int M = batch.M;
    const int64_t total = (int64_t)M * P.N;
    const int64_t e = ((int64_t)(blockIdx.x - P.red_begin) * 256 + threadIdx.x) * 4;
    if (P.splits <= 1 || e >= total) return;
    const float* base = ws + P.ws_off + e;
    if ((P.N & 3) == 0) {  // 4 elements of one row
        const f32x4 v = sum_planes(base, total, P.splits);
        const int row = (int)(e / P.N), col = (int)(e % P.N);
#pragma unroll
        for (int c = 0; c < 4; ++c) P.C[(int64_t)row * P.ldc + col + c] = f32_to_bf16(epi_fn(P.epi, v[c]));
        return;
    }
    for (int c = 0; c < 4 && e + c < total; ++c) {
        float v = base[c];
        for (int s = 1; s < P.splits; ++s) v += base[c + s * total];
        const int row = (int)((e + c) / P.N), col = (int)((e + c) % P.N);
        P.C[(int64_t)row * P.ldc + col] = f32_to_bf16(epi_fn(P.epi, v));
    }
}

// Pack an nn.Linear weight B [N][K] (row stride ldb) into 64 x 64 tiles: tile
// (nt, kt) is the 8 KB block at ((nt * KT) + kt) * 4096 elements, row r of it
// holds B[64 nt + r][64 kt .. +63] as 8 chunks of 16 bytes with logical chunk
// c at position c ^ swz(r); rows past N and columns past K are zero.
__global__ __launch_bounds__(256) void gemm_pack_kernel(const bf16_t* __restrict__ B, int64_t ldb, int N, int K,
                                                        int KT, int64_t chunks, bf16_t* __restrict__ out) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= chunks) return;
    const int p = (int)(q & 7), r = (int)((q >> 3) & 63);
    const int64_t tile = q >> 9;
    const int kt = (int)(tile % KT), nt = (int)(tile / KT);
    const int n = nt * 64 + r, k = kt * 64 + 8 * (p ^ swz(r));
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (n < N && k < K) v = *reinterpret_cast<const uint4*>(B + (int64_t)n * ldb + k);
    reinterpret_cast<uint4*>(out)[q] = v;
}

// Launch plan of a problem set on a bm x bn tile: split counts (when the tiles
// alone would not reach `target` blocks, K splits into equal ranges of at least
// min_k, a multiple of BK, at most 8), block offsets, workspace floats and the
// tiles the reduction pass covers.  force_splits > 0 overrides the split rule.
struct Plan {
    int splits[kMaxProblems], k_per[kMaxProblems];
    int blocks, red_tiles;  // blocks of the GEMM and of the reduction pass
    int64_t ws_floats;
};

Plan make_plan(int bm, int bn, int M, int count, const int* N, const int* K, int target, int min_k,
               int force_splits) {
    Plan pl{};
    const int mt = (M + bm - 1) / bm;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) total += (int64_t)mt * ((N[i] + bn - 1) / bn);
    const int want = (int)((target + total - 1) / total);
    for (int i = 0; i < count; ++i) {
        const int n_tiles = (N[i] + bn - 1) / bn;
        int si = force_splits > 0 ? force_splits : want;
        if (force_splits <= 0) {
            const int max_by_k = K[i] / min_k;
            if (si > max_by_k) si = max_by_k < 1 ? 1 : max_by_k;
            if (si > 8) si = 8;
        }
        if (si < 1) si = 1;
        int kp = (K[i] + si - 1) / si;
        kp = (kp + BK - 1) / BK * BK;
        si = (K[i] + kp - 1) / kp;
        pl.splits[i] = si;
        pl.k_per[i] = kp;
        pl.blocks += 8 * ((n_tiles + 7) / 8) * mt * si;
        if (si > 1) {
            pl.ws_floats += (int64_t)si * M * N[i];
            pl.red_tiles += (int)((((int64_t)M * N[i] + 3) / 4 + 255) / 256);
        }
    }
    return pl;
}

template <class T>
hipError_t launch_tile(int M, int count, const void* const* A, const void* const* B, void* const* C,
                       const int64_t* lda, const int64_t* ldc, const int* N, const int* K,
                       const int* epi, float* ws, hipStream_t st, const Plan& pl, int partial = 0) {
    GemmBatch b{};
    b.count = count;
    b.M = M;
    b.bm = T::BM;
    b.bn = T::BN;
    const int mt = (M + T::BM - 1) / T::BM;
    int blocks = 0, red = 0;
    int64_t ws_off = 0;
    for (int i = 0; i < count; ++i) {
        GemmProblem& p = b.p[i];
        p.A = (const bf16_t*)A[i];
        p.B = (const bf16_t*)B[i];
        p.C = (bf16_t*)C[i];
        p.lda = lda[i];
        p.ldc = ldc[i];
        p.N = N[i];
        p.K = K[i];
        p.epi = epi[i];
        p.n_tiles = (N[i] + T::BN - 1) / T::BN;
        p.k_tiles = (K[i] + BK - 1) / BK;
        p.n64 = (N[i] + 63) / 64;
        p.splits = pl.splits[i];
        p.k_per = pl.k_per[i];
        p.block_begin = blocks;
        p.ws_off = ws_off;
        p.red_begin = red;
        blocks += 8 * ((p.n_tiles + 7) / 8) * mt * p.splits;
        p.partial = partial;
        if (p.splits > 1 || partial) {
            ws_off += (int64_t)p.splits * M * N[i];
            if (!partial) red += (int)((((int64_t)M * N[i] + 3) / 4 + 255) / 256);
        }
    }
    hipLaunchKernelGGL((gemm_decode_kernel<T>), dim3(blocks), dim3(T::THREADS), 0, st, b, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || red == 0 || partial) return e;
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3(red), dim3(256), 0, st, b, (const float*)ws);
    return hipGetLastError();
}

// Tiles and K splits by row count, chosen by a sweep of tiles (32 x 32 to
// 256 x 32, 64 x 64, 128 x 64; 4 to 16 waves) and block targets (1 to 512)
// over the five launches of a 1.5B and a 7.2B decode layer at M = 32 .. 256,
// cold weights (MI355X; the plans compared in one process, interleaved):
//   * up to 32 rows a 32 x 32 tile (4 K groups) with K split to about 256
//     blocks (summed by the reduction launch): every block only streams
//     weights, and the narrow tile gives twice the column tiles and half the
//     dead activation rows;
//   * above 32 rows, results the kernel writes itself (epilogue applied) are
//     not split (the reduction launch costs more than the split gains: 1.5B
//     layer at 40-64 rows 86 -> 74-81 us without it), and their tile minimises
//     ceil(blocks / CUs) x (BM + BN): the rounds of blocks a CU runs times the
//     rows and columns each block streams per K step (a CU's loads, not the
//     matrix cores, bound these launches); ties go to the smaller tile, which
//     puts more blocks on the CUs.  Measured per launch (graph replays over the
//     layers): a 1.5B layer's r/k/v + LoRA-down and FFN key launches at 40-64
//     rows 16.2-17.3 -> 14.4-16.3 us (32 x 32 instead of 64 x 64), at 80-128
//     rows 18.8-20.2 -> 16.8-17.6 us (64 x 64 instead of 128 x 64, which left
//     half the CUs idle), unchanged above; a 7.2B layer keeps 64 x 64 up to 64
//     rows and 128 x 64 up to 128 (its wider matrices fill the GPU), and at
//     160 rows takes 64 x 64 (55.6 / 62.5 against 61.0 / 65.7 us);
//   * partial planes (summed by the next row kernel, no reduction launch):
//     64 x 64 up to 64 rows, 128 x 64 above (one row tile up to 128 rows, so
//     each weight tile is read once), split to about 512 blocks up to 128 rows
//     and 256 above.
using TileNarrow = Tile<1, 1, 1, 1, 4, 4>;
using TileDecode = Tile<2, 2, 1, 1, 4, 2>;
using TileWide = Tile<4, 2, 1, 1, 4, 1>;
constexpr int kMinK = 512;

enum TileKind { kNarrow, kDecode, kWide };

// compute units of the current device (queried once per device)
int cu_count() {
    static std::mutex mu;
    static int cached[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

TileKind tile_for(int M, bool partial, int count, const int* N) {
    if (M <= 32) return kNarrow;
    if (partial) return M <= 64 ? kDecode : kWide;
    const int cus = cu_count();
    const int bm[3] = {TileNarrow::BM, TileDecode::BM, TileWide::BM};
    const int bn[3] = {TileNarrow::BN, TileDecode::BN, TileWide::BN};
    TileKind best = kNarrow;
    int64_t best_cost = -1;
    for (int t = 0; t < 3; ++t) {
        int64_t blocks = 0;
        for (int i = 0; i < count; ++i) blocks += (int64_t)((N[i] + bn[t] - 1) / bn[t]) * ((M + bm[t] - 1) / bm[t]);
        const int64_t cost = (blocks + cus - 1) / cus * (bm[t] + bn[t]);
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = (TileKind)t;
        }
    }
    return best;
}

int target_for(int M, bool partial) {
    if (partial) return M <= 128 ? 512 : 256;
    return M <= 32 ? 256 : 1;
}

Plan plan_for(int M, int count, const int* N, const int* K, bool partial) {
    const int target = target_for(M, partial);
    switch (tile_for(M, partial, count, N)) {
        case kNarrow: return make_plan(TileNarrow::BM, TileNarrow::BN, M, count, N, K, target, kMinK, 0);
        case kDecode: return make_plan(TileDecode::BM, TileDecode::BN, M, count, N, K, target, kMinK, 0);
        default: return make_plan(TileWide::BM, TileWide::BN, M, count, N, K, target, kMinK, 0);
    }
}

hipError_t launch_for(int M, int count, const void* const* A, const void* const* B, void* const* C,
                      const int64_t* lda, const int64_t* ldc, const int* N, const int* K, const int* epi, float* ws,
                      hipStream_t st, int partial) {
    const Plan pl = plan_for(M, count, N, K, partial != 0);
    switch (tile_for(M, partial != 0, count, N)) {
        case kNarrow: return launch_tile<TileNarrow>(M, count, A, B, C, lda, ldc, N, K, epi, ws, st, pl, partial);
        case kDecode: return launch_tile<TileDecode>(M, count, A, B, C, lda, ldc, N, K, epi, ws, st, pl, partial);
        default: return launch_tile<TileWide>(M, count, A, B, C, lda, ldc, N, K, epi, ws, st, pl, partial);
    }
}

}  // namespace

int gemm_decode_max_problems() { return kMaxProblems; }

int64_t gemm_decode_workspace(int M, int count, const int* N, const int* K) {
    return plan_for(M, count, N, K, false).ws_floats;
}

// problems: count entries of {A, packed B, C, lda, ldc, N, K, epi}
hipError_t launch_gemm_decode(int M, int count, const void* const* A, const void* const* B, void* const* C,
                              const int64_t* lda, const int64_t* ldc, const int* N, const int* K,
                              const int* epi, float* ws, hipStream_t st)
{
    return launch_for(M, count, A, B, C, lda, ldc, N, K, epi, ws, st, 0);
}

// One problem, its K-range partial products left as float32 [splits][M][N] rows
// at the start of ws (no epilogue, no reduction pass; one range when the plan
// does not split).  Their in-order sum rounded to bf16 is the product with
// epi 0 (launch_gemm_decode may split it differently).
int gemm_decode_partial_splits(int M, int N, int K) { return plan_for(M, 1, &N, &K, true).splits[0]; }

hipError_t launch_gemm_decode_partials(int M, const void* A, const void* B, int64_t lda, int N, int K, float* ws,
                                       hipStream_t st)
{
    void* C = nullptr;
    const int64_t ldc = N;
    const int epi = 0;
    return launch_for(M, 1, &A, &B, &C, &lda, &ldc, &N, &K, &epi, ws, st, 1);
}

int64_t gemm_packed_elems(int N, int K) { return (int64_t)((N + 63) / 64) * 64 * ((K + BK - 1) / BK) * BK; }

hipError_t launch_gemm_pack(const void* B, int64_t ldb, int N, int K, void* out, hipStream_t st) {
    const int KT = (K + BK - 1) / BK;
    const int64_t chunks = gemm_packed_elems(N, K) / 8;
    hipLaunchKernelGGL(gemm_pack_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st,
                       (const bf16_t*)B, ldb, N, K, KT, chunks, (bf16_t*)out);
    return hipGetLastError();
}
